/*
 * ORACLE — test infrastructure only. Not part of the product.
 *
 * Plain-C restatement of the reference BigSmall CPU encode/decode algorithms
 * for the rANS-family bf16 codecs. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline legs of bench.py may load this library: to check results
 * against, as the timed CPU baseline, and to write the reference-format blobs
 * that baseline decodes. The product decode path (bigsmall_amd) never links
 * or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference repository root). Pinning (see tests/test_oracle_*.py):
 *   - orc_quantise_ref / orc_quantise_sk / orc_rans_encode / orc_rans_decode,
 *     orc_par1_*, orc_tans_*, orc_sk_*: byte-for-byte against golden vectors
 *     written by tests/golden/make_golden.py from the reference's own
 *     pure-Python modules, plus closed forms (single-symbol stream =
 *     "00 00 01 00", empty tensor -> empty blob) and brute-force round trips.
 *   - orc_chunk_decode (the build's own GPU-native container format, which has
 *     no reference counterpart): pinned by lossless round trips against the
 *     source tensors' md5 and hand-built tiny blobs.
 *
 * All integers little-endian. Status codes: 0 ok, <0 error.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_OK 0
#define ORC_ERR_ARG -1
#define ORC_ERR_FORMAT -2
#define ORC_ERR_CAP -3
#define ORC_ERR_QUANT -4
#define ORC_ERR_COUNT -5

#define RANS_L (1u << 16)

/* ------------------------------------------------------------------------ */
/* little-endian helpers                                                     */

static inline void put16(uint8_t *p, uint32_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
static inline void put32(uint8_t *p, uint32_t v) {
    p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); p[2] = (uint8_t)(v >> 16); p[3] = (uint8_t)(v >> 24);
}
static inline uint32_t get16(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }
static inline uint32_t get32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static inline uint64_t get64(const uint8_t *p) { return (uint64_t)get32(p) | ((uint64_t)get32(p + 4) << 32); }

typedef struct { uint8_t *p; size_t len, cap; int err; } wbuf;
static void wb_put(wbuf *w, const void *src, size_t n) {
    if (w->err) return;
    if (w->len + n > w->cap) { w->err = 1; return; }
    memcpy(w->p + w->len, src, n); w->len += n;
}
static void wb_u8(wbuf *w, uint32_t v) { uint8_t b = (uint8_t)v; wb_put(w, &b, 1); }
static void wb_u16(wbuf *w, uint32_t v) { uint8_t b[2]; put16(b, v); wb_put(w, b, 2); }
static void wb_u32(wbuf *w, uint32_t v) { uint8_t b[4]; put32(b, v); wb_put(w, b, 4); }

typedef struct { const uint8_t *p; size_t len, pos; int err; } rbuf;
/* io.BytesIO.read semantics: returns what is there; a short read flags err */
static const uint8_t *rb_take(rbuf *r, size_t n) {
    if (r->err || r->pos + n > r->len) { r->err = 1; return NULL; }
    const uint8_t *q = r->p + r->pos; r->pos += n; return q;
}
static uint32_t rb_u8(rbuf *r) { const uint8_t *q = rb_take(r, 1); return q ? q[0] : 0; }
static uint32_t rb_u16(rbuf *r) { const uint8_t *q = rb_take(r, 2); return q ? get16(q) : 0; }
static uint32_t rb_u32(rbuf *r) { const uint8_t *q = rb_take(r, 4); return q ? get32(q) : 0; }

/* ------------------------------------------------------------------------ */
/* Frequency quantisation                                                    */

/* bigsmall/codecs/rans.py:34-92 (identical algorithm in
 * bigsmall/codecs/numba_rans.py:45-85). Floor-scale, force >=1 for nonzero,
 * then +/-1 round-robin over np.argsort(-scaled, kind="stable"). */
int orc_quantise_ref(const int64_t *counts, int alphabet, uint32_t M, uint32_t *out) {
    if (alphabet <= 0) return ORC_ERR_ARG;
    int64_t *sc = (int64_t *)malloc(sizeof(int64_t) * alphabet);
    int *order = (int *)malloc(sizeof(int) * alphabet);
    if (!sc || !order) { free(sc); free(order); return ORC_ERR_ARG; }
    int n_nz = 0; int64_t total = 0;
    for (int i = 0; i < alphabet; i++) if (counts[i] > 0) { n_nz++; total += counts[i]; }
    /* rans.py:49-54: all mass on symbol 0 */
    if (n_nz == 0) {
        for (int i = 0; i < alphabet; i++) out[i] = 0;
        out[0] = M; free(sc); free(order); return ORC_OK;
    }
    if ((uint32_t)n_nz > M) { free(sc); free(order); return ORC_ERR_QUANT; }
    /* rans.py:61-67. counts are int64; total = counts.sum() (all entries) */
    total = 0; for (int i = 0; i < alphabet; i++) total += counts[i];
    int64_t sum = 0;
    for (int i = 0; i < alphabet; i++) {
        int64_t v = (counts[i] * (int64_t)M) / total;   /* floor: counts >= 0 */
        if (counts[i] > 0 && v < 1) v = 1;
        if (counts[i] == 0) v = 0;
        sc[i] = v; sum += v;
    }
    int64_t diff = (int64_t)M - sum;
    if (diff != 0) {
        /* np.argsort(-scaled, kind="stable"): descending by value, ties by index.
         * Insertion sort is stable and alphabet is small (<= 512). */
        for (int i = 0; i < alphabet; i++) {
            int j = i; order[j] = i;
            while (j > 0 && -sc[order[j - 1]] > -sc[i]) { order[j] = order[j - 1]; j--; }
            order[j] = i;
        }
    }
    if (diff > 0) {
        int64_t i = 0;                                   /* rans.py:70-77 */
        while (diff > 0) { sc[order[i % alphabet]] += 1; diff--; i++; }
    } else if (diff < 0) {
        int64_t i = 0;                                   /* rans.py:78-90 */
        while (diff < 0) {
            int j = order[i % alphabet];
            if (sc[j] > 1) { sc[j] -= 1; diff++; }
            i++;
            if (i > 100 * (int64_t)alphabet) { free(sc); free(order); return ORC_ERR_QUANT; }
        }
    }
    for (int i = 0; i < alphabet; i++) out[i] = (uint32_t)sc[i];
    free(sc); free(order);
    return ORC_OK;
}

/* bigsmall/codecs/single_kernel.py:53-110 (_quantise_inplace): floor-scale with
 * min 1, then repeatedly +1 on the first argmax (strict '>' scan), or -1 on
 * the first argmax while it is > 1 (bounded by 50*alphabet iterations). */
int orc_quantise_sk(const int64_t *counts, int alphabet, uint32_t M, uint32_t *out) {
    int n_nz = 0; int64_t total = 0;
    for (int i = 0; i < alphabet; i++) if (counts[i] > 0) { n_nz++; total += counts[i]; }
    if (n_nz == 0) {
        for (int i = 0; i < alphabet; i++) out[i] = 0;
        out[0] = M; return ORC_OK;
    }
    int64_t s = 0;
    for (int i = 0; i < alphabet; i++) {
        if (counts[i] > 0) {
            int64_t v = (counts[i] * (int64_t)M) / total;
            if (v < 1) v = 1;
            out[i] = (uint32_t)v; s += v;
        } else out[i] = 0;
    }
    int64_t diff = (int64_t)M - s;
    if (diff > 0) {
        while (diff > 0) {
            int best = 0; uint32_t bv = 0;
            for (int i = 0; i < alphabet; i++) if (out[i] > bv) { bv = out[i]; best = i; }
            out[best] += 1; diff--;
        }
    } else if (diff < 0) {
        int guard = 0;
        while (diff < 0 && guard < 50 * alphabet) {
            int best = 0; uint32_t bv = 0;
            for (int i = 0; i < alphabet; i++) if (out[i] > bv) { bv = out[i]; best = i; }
            if (out[best] > 1) { out[best] -= 1; diff++; } else break;
            guard++;
        }
    }
    return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* rANS stream primitive                                                     */

static int log2_pow2(uint32_t M) {
    if (M == 0 || (M & (M - 1))) return -1;
    int p = 0; while ((1u << p) != M) p++; return p;
}

/* bigsmall/codecs/rans.py:115-162 (byte-identical to numba_rans.py:108-164 and
 * single_kernel.py:121-156 + its reversal). Output: [u32 final state][u16 words
 * in decode order]. Empty input -> the 4-byte state L. */
int64_t orc_rans_encode(const int32_t *syms, size_t n, const uint32_t *freqs, int alphabet,
                        uint32_t M, uint8_t *out, size_t cap) {
    if (log2_pow2(M) < 0) return ORC_ERR_ARG;
    if (n == 0) { if (cap < 4) return ORC_ERR_CAP; put32(out, RANS_L); return 4; }
    uint32_t *cum = (uint32_t *)malloc(sizeof(uint32_t) * alphabet);
    uint16_t *stack = (uint16_t *)malloc(sizeof(uint16_t) * (n + 4));
    if (!cum || !stack) { free(cum); free(stack); return ORC_ERR_ARG; }
    uint32_t c = 0;
    for (int i = 0; i < alphabet; i++) { cum[i] = c; c += freqs[i]; }
    uint64_t state = RANS_L, state_max = 1ull << 32;
    size_t ns = 0;
    for (size_t ii = n; ii-- > 0;) {
        int s = syms[ii];
        if (s < 0 || s >= alphabet || freqs[s] == 0) { free(cum); free(stack); return ORC_ERR_ARG; }
        uint64_t f = freqs[s], cf = cum[s];
        uint64_t upper = (state_max / M) * f;
        while (state >= upper) {
            if (ns >= n + 4) { free(cum); free(stack); return ORC_ERR_FORMAT; }
            stack[ns++] = (uint16_t)(state & 0xFFFF); state >>= 16;
        }
        state = (state / f) * M + cf + (state % f);
        if (state >= state_max) { free(cum); free(stack); return ORC_ERR_FORMAT; }
    }
    size_t need = 4 + 2 * ns;
    if (need > cap) { free(cum); free(stack); return ORC_ERR_CAP; }
    put32(out, (uint32_t)state);
    for (size_t k = 0; k < ns; k++) put16(out + 4 + 2 * k, stack[ns - 1 - k]);
    free(cum); free(stack);
    return (int64_t)need;
}

/* bigsmall/codecs/rans.py:165-207 decode_stream, including its tail rule:
 * renormalise while state < L and bytes remain; if exactly one byte remains,
 * shift in zeros and stop reading (rans.py:196-202). */
int orc_rans_decode(const uint8_t *data, size_t len, size_t n, const uint32_t *freqs, int alphabet,
                    uint32_t M, uint32_t *out) {
    if (n == 0) return ORC_OK;
    if (len < 4) return ORC_ERR_FORMAT;
    int p = log2_pow2(M); if (p < 0) return ORC_ERR_ARG;
    uint32_t *cum = (uint32_t *)malloc(sizeof(uint32_t) * alphabet);
    uint16_t *tbl = (uint16_t *)calloc(M, sizeof(uint16_t));
    if (!cum || !tbl) { free(cum); free(tbl); return ORC_ERR_ARG; }
    uint32_t c = 0;
    for (int i = 0; i < alphabet; i++) { cum[i] = c; c += freqs[i]; }
    /* rans.py:102-112 build_slot_to_symbol */
    for (int s = 0; s < alphabet; s++)
        for (uint32_t k = 0; k < freqs[s] && cum[s] + k < M; k++) tbl[cum[s] + k] = (uint16_t)s;
    uint64_t state = get32(data);   /* Python int: unbounded */
    size_t pos = 4;
    for (size_t i = 0; i < n; i++) {
        uint32_t slot = (uint32_t)(state & (M - 1));
        uint32_t s = tbl[slot];
        out[i] = s;
        state = (uint64_t)freqs[s] * (state >> p) + slot - cum[s];
        while (state < RANS_L && pos + 1 < len + 1) {
            if (pos + 2 > len) { state <<= 16; pos = len; break; }
            state = (state << 16) | get16(data + pos); pos += 2;
        }
    }
    free(cum); free(tbl);
    return ORC_OK;
}

/* bigsmall/codecs/numba_rans.py:167-217 decode_stream/_decode_kernel: odd-length
 * data is zero-padded to a whole u16; state = u16[0] | u16[1] << 16 in uint32
 * arithmetic; renormalise while state < L and u16s remain. `start_u16` lets the
 * same loop serve single_kernel.py:159-190 (_rans_decode_one). */
static void nb_decode_u16(const uint16_t *d, size_t n_u16, size_t n, const uint32_t *freqs,
                          const uint32_t *cum, const uint32_t *tbl, int prec, uint32_t *out) {
    uint32_t state = (uint32_t)d[0] | ((uint32_t)d[1] << 16);
    size_t pos = 2;
    uint32_t mask = (1u << prec) - 1;
    for (size_t i = 0; i < n; i++) {
        uint32_t slot = state & mask;
        uint32_t s = tbl[slot];
        out[i] = s;
        state = freqs[s] * (state >> prec) + slot - cum[s];
        while (state < RANS_L && pos < n_u16) { state = (state << 16) | d[pos]; pos++; }
    }
}

static int nb_decode_bytes(const uint8_t *data, size_t len, size_t n, const uint32_t *freqs,
                           int alphabet, int prec, uint32_t *out) {
    if (n == 0) return ORC_OK;
    if (len < 4) return ORC_ERR_FORMAT;
    uint32_t M = 1u << prec;
    size_t n_u16 = (len + 1) / 2;
    uint16_t *d = (uint16_t *)calloc(n_u16 + 1, sizeof(uint16_t));
    uint32_t *cum = (uint32_t *)malloc(sizeof(uint32_t) * alphabet);
    uint32_t *tbl = (uint32_t *)calloc(M, sizeof(uint32_t));
    if (!d || !cum || !tbl) { free(d); free(cum); free(tbl); return ORC_ERR_ARG; }
    for (size_t i = 0; i < len; i++) d[i / 2] |= (uint16_t)((uint32_t)data[i] << (8 * (i & 1)));
    uint32_t c = 0;
    for (int i = 0; i < alphabet; i++) { cum[i] = c; c += freqs[i]; }
    /* numba_rans.py:95-102 slot_to_symbol_table */
    for (int s = 0; s < alphabet; s++)
        for (uint32_t k = 0; k < freqs[s] && cum[s] + k < M; k++) tbl[cum[s] + k] = (uint32_t)s;
    nb_decode_u16(d, n_u16, n, freqs, cum, tbl, prec, out);
    free(d); free(cum); free(tbl);
    return ORC_OK;
}

int orc_rans_decode_nb(const uint8_t *data, size_t len, size_t n, const uint32_t *freqs, int alphabet,
                       int prec, uint32_t *out) {
    return nb_decode_bytes(data, len, n, freqs, alphabet, prec, out);
}

/* ------------------------------------------------------------------------ */
/* bf16 helpers (bigsmall/codecs/bf16.py:25-30)                              */

#define SE_ALPHABET 512
#define MANT_ALPHABET 128

static inline uint32_t w_sign(uint16_t w) { return (w >> 15) & 1; }
static inline uint32_t w_exp(uint16_t w) { return (w >> 7) & 0xFF; }
static inline uint32_t w_mant(uint16_t w) { return w & 0x7F; }

/* Stable counting sort of the positions of `exp` (np.argsort(kind="stable")
 * on uint16 exponents): order[k] = index of the k-th element in sorted order. */
static void stable_order_by_exp(const uint32_t *exp, size_t n, size_t *order, int64_t *bstart) {
    int64_t cnt[256] = {0};
    for (size_t i = 0; i < n; i++) cnt[exp[i]]++;
    bstart[0] = 0;
    for (int e = 0; e < 256; e++) bstart[e + 1] = bstart[e] + cnt[e];
    int64_t cur[256];
    for (int e = 0; e < 256; e++) cur[e] = bstart[e];
    for (size_t i = 0; i < n; i++) order[cur[exp[i]]++] = i;
}

/* ------------------------------------------------------------------------ */
/* bf16_parallel_v1  (bigsmall/codecs/bf16_parallel.py)                      */

#define PAR_PREC_SE 12
#define PAR_PREC_M 10

/* bf16_parallel.py:186-259 encode. Returns bytes written or <0. */
int64_t orc_par1_encode(const uint16_t *w, size_t n, int n_streams_req, uint8_t *out, size_t cap) {
    if (n == 0) return 0;                                   /* :192-193 */
    if (n > 0xFFFFFFFFull) return ORC_ERR_ARG;
    int N = n_streams_req;
    if ((size_t)N > n) N = (int)n;
    if (N < 1) N = 1;                                       /* :195 */
    if (N > 0xFFFF) return ORC_ERR_ARG;
    int rc = ORC_OK;
    wbuf wb = {out, 0, cap, 0};
    uint32_t *se = (uint32_t *)malloc(sizeof(uint32_t) * n);
    uint32_t *ex = (uint32_t *)malloc(sizeof(uint32_t) * n);
    int64_t (*mcnt)[MANT_ALPHABET] = (int64_t (*)[MANT_ALPHABET])calloc(256, sizeof(*mcnt));
    uint32_t (*mfreq)[MANT_ALPHABET] = (uint32_t (*)[MANT_ALPHABET])calloc(256, sizeof(*mfreq));
    if (!se || !ex || !mcnt || !mfreq) { free(se); free(ex); free(mcnt); free(mfreq); return ORC_ERR_ARG; }
    int64_t se_cnt[SE_ALPHABET] = {0}, exp_cnt[256] = {0};
    for (size_t i = 0; i < n; i++) {
        se[i] = (w_sign(w[i]) << 8) | w_exp(w[i]); ex[i] = w_exp(w[i]);
        se_cnt[se[i]]++; exp_cnt[ex[i]]++; mcnt[ex[i]][w_mant(w[i])]++;
    }
    /* :77-103 _build_shared_freqs */
    uint32_t se_freqs[SE_ALPHABET];
    if ((rc = orc_quantise_ref(se_cnt, SE_ALPHABET, 1u << PAR_PREC_SE, se_freqs)) != ORC_OK) goto done;
    for (int e = 0; e < 256; e++)
        if (exp_cnt[e] && (rc = orc_quantise_ref(mcnt[e], MANT_ALPHABET, 1u << PAR_PREC_M, mfreq[e])) != ORC_OK) goto done;

    /* :106-135 _pack_header */
    wb_put(&wb, "PAR1", 4);
    wb_u32(&wb, (uint32_t)n); wb_u16(&wb, (uint32_t)N); wb_u16(&wb, PAR_PREC_SE); wb_u16(&wb, PAR_PREC_M);
    int n_se_nz = 0; for (int s = 0; s < SE_ALPHABET; s++) if (se_freqs[s]) n_se_nz++;
    wb_u16(&wb, (uint32_t)n_se_nz);
    for (int s = 0; s < SE_ALPHABET; s++) if (se_freqs[s]) wb_u16(&wb, (uint32_t)s);
    for (int s = 0; s < SE_ALPHABET; s++) if (se_freqs[s]) wb_u32(&wb, se_freqs[s]);
    int n_exps = 0; for (int e = 0; e < 256; e++) if (exp_cnt[e]) n_exps++;
    wb_u32(&wb, (uint32_t)n_exps);
    for (int e = 0; e < 256; e++) if (exp_cnt[e]) wb_u16(&wb, (uint32_t)e);
    for (int e = 0; e < 256; e++) {
        if (!exp_cnt[e]) continue;
        int k = 0; for (int m = 0; m < MANT_ALPHABET; m++) if (mfreq[e][m]) k++;
        wb_u8(&wb, (uint32_t)k);
        for (int m = 0; m < MANT_ALPHABET; m++) if (mfreq[e][m]) wb_u8(&wb, (uint32_t)m);
        for (int m = 0; m < MANT_ALPHABET; m++) if (mfreq[e][m]) wb_u32(&wb, mfreq[e][m]);
    }
    size_t off_pos = wb.len;
    for (int k = 0; k <= N; k++) wb_u32(&wb, 0);             /* patched below */
    if (wb.err) { rc = ORC_ERR_CAP; goto done; }
    size_t payload_start = wb.len;

    size_t per = (n + N - 1) / N;
    int32_t *sym = (int32_t *)malloc(sizeof(int32_t) * per);
    uint32_t *esl = (uint32_t *)malloc(sizeof(uint32_t) * per);
    size_t *order = (size_t *)malloc(sizeof(size_t) * per);
    int32_t *bucket = (int32_t *)malloc(sizeof(int32_t) * per);
    if (!sym || !esl || !order || !bucket) { free(sym); free(esl); free(order); free(bucket); rc = ORC_ERR_ARG; goto done; }
    for (int k = 0; k < N; k++) {
        put32(out + off_pos + 4 * k, (uint32_t)(wb.len - payload_start));
        size_t cnt = 0;
        for (size_t i = (size_t)k; i < n; i += N) { sym[cnt] = (int32_t)se[i]; esl[cnt] = ex[i]; cnt++; }
        /* :213-235 (cnt > 0 always since N <= n) */
        size_t lenpos = wb.len; wb_u32(&wb, 0);
        if (wb.err) break;
        int64_t bl = orc_rans_encode(sym, cnt, se_freqs, SE_ALPHABET, 1u << PAR_PREC_SE, wb.p + wb.len, wb.cap - wb.len);
        if (bl < 0) { rc = (int)bl; break; }
        put32(out + lenpos, (uint32_t)bl); wb.len += (size_t)bl;
        int64_t bstart[257];
        stable_order_by_exp(esl, cnt, order, bstart);
        int m = 0; for (int e = 0; e < 256; e++) if (bstart[e + 1] > bstart[e]) m++;
        wb_u32(&wb, (uint32_t)m);
        for (int e = 0; e < 256; e++) if (bstart[e + 1] > bstart[e]) wb_u16(&wb, (uint32_t)e);
        for (int e = 0; e < 256 && !wb.err; e++) {
            if (bstart[e + 1] == bstart[e]) continue;
            size_t bc = (size_t)(bstart[e + 1] - bstart[e]);
            for (size_t j = 0; j < bc; j++) bucket[j] = (int32_t)w_mant(w[(size_t)k + order[bstart[e] + j] * N]);
            size_t hdr = wb.len; wb_u32(&wb, 0); wb_u32(&wb, 0);
            if (wb.err) break;
            int64_t ml = orc_rans_encode(bucket, bc, mfreq[e], MANT_ALPHABET, 1u << PAR_PREC_M, wb.p + wb.len, wb.cap - wb.len);
            if (ml < 0) { rc = (int)ml; break; }
            put32(out + hdr, (uint32_t)bc); put32(out + hdr + 4, (uint32_t)ml); wb.len += (size_t)ml;
        }
        if (rc != ORC_OK || wb.err) break;
    }
    free(sym); free(esl); free(order); free(bucket);
    if (rc == ORC_OK && wb.err) rc = ORC_ERR_CAP;
    if (rc == ORC_OK) put32(out + off_pos + 4 * N, (uint32_t)(wb.len - payload_start));
done:
    free(se); free(ex); free(mcnt); free(mfreq);
    return rc == ORC_OK ? (int64_t)wb.len : rc;
}

/* Shared parse of the PAR1 header: bf16_parallel.py:138-183 _unpack_header. */
typedef struct {
    uint32_t n, N;
    uint32_t se_freqs[SE_ALPHABET];
    int n_exps; uint32_t exps[256];
    uint32_t mfreq[256][MANT_ALPHABET];
    size_t header_end;
} par1_hdr;

static int par1_parse(const uint8_t *blob, size_t len, par1_hdr *h) {
    rbuf r = {blob, len, 0, 0};
    const uint8_t *mg = rb_take(&r, 4);
    if (!mg || memcmp(mg, "PAR1", 4) != 0) return ORC_ERR_FORMAT;
    h->n = rb_u32(&r); h->N = rb_u16(&r);
    uint32_t pse = rb_u16(&r), pm = rb_u16(&r);
    if (r.err || pse != PAR_PREC_SE || pm != PAR_PREC_M) return ORC_ERR_FORMAT;
    memset(h->se_freqs, 0, sizeof(h->se_freqs));
    uint32_t nnz = rb_u16(&r);
    const uint8_t *idx = rb_take(&r, 2 * (size_t)nnz), *fq = rb_take(&r, 4 * (size_t)nnz);
    if (r.err) return ORC_ERR_FORMAT;
    for (uint32_t i = 0; i < nnz; i++) {
        uint32_t s = get16(idx + 2 * i); if (s >= SE_ALPHABET) return ORC_ERR_FORMAT;
        h->se_freqs[s] = get32(fq + 4 * i);
    }
    uint32_t ne = rb_u32(&r);
    if (r.err || ne > 256) return ORC_ERR_FORMAT;
    h->n_exps = (int)ne;
    const uint8_t *ev = rb_take(&r, 2 * (size_t)ne);
    if (r.err) return ORC_ERR_FORMAT;
    for (uint32_t i = 0; i < ne; i++) { h->exps[i] = get16(ev + 2 * i); if (h->exps[i] > 255) return ORC_ERR_FORMAT; }
    memset(h->mfreq, 0, sizeof(h->mfreq));
    for (uint32_t i = 0; i < ne; i++) {
        uint32_t k = rb_u8(&r);
        const uint8_t *mi = rb_take(&r, k), *mf = rb_take(&r, 4 * (size_t)k);
        if (r.err) return ORC_ERR_FORMAT;
        for (uint32_t j = 0; j < k; j++) {
            if (mi[j] >= MANT_ALPHABET) return ORC_ERR_FORMAT;
            h->mfreq[h->exps[i]][mi[j]] = get32(mf + 4 * j);
        }
    }
    h->header_end = r.pos;
    return ORC_OK;
}

/* bf16_parallel.py:262-352 decode. */
/* Streams [k0, k1) of the blob (clamped to its N); each stream writes only
 * its own elements k, k + N, ... of `out`, so disjoint ranges may run on
 * separate threads (the reference decodes its streams one after another,
 * bf16_parallel.py:298-351). */
int orc_par1_decode_streams(const uint8_t *blob, size_t len, size_t n_weights, uint16_t *out, size_t k0,
                            size_t k1) {
    if (n_weights == 0 || len == 0) return ORC_OK;          /* :268-269 */
    par1_hdr *h = (par1_hdr *)malloc(sizeof(par1_hdr));
    if (!h) return ORC_ERR_ARG;
    int rc = par1_parse(blob, len, h);
    if (rc) { free(h); return rc; }
    if (h->n != n_weights || h->N == 0) { free(h); return ORC_ERR_COUNT; }
    size_t n = h->n, N = h->N;
    size_t off_end = h->header_end + 4 * (N + 1);
    if (off_end > len) { free(h); return ORC_ERR_FORMAT; }
    size_t per = (n + N - 1) / N;
    uint32_t *se = (uint32_t *)malloc(sizeof(uint32_t) * per);
    uint32_t *ms = (uint32_t *)malloc(sizeof(uint32_t) * per);
    uint32_t *tmp = (uint32_t *)malloc(sizeof(uint32_t) * per);
    size_t *order = (size_t *)malloc(sizeof(size_t) * per);
    if (!se || !ms || !tmp || !order) { rc = ORC_ERR_ARG; goto out; }
    if (k1 > N) k1 = N;
    for (size_t k = k0; k < k1; k++) {
        size_t nk = k < n ? (n - 1 - k) / N + 1 : 0;         /* :293-296 */
        if (nk == 0) continue;
        size_t a = get32(blob + h->header_end + 4 * k), b = get32(blob + h->header_end + 4 * (k + 1));
        if (a > b || off_end + b > len) { rc = ORC_ERR_FORMAT; break; }
        rbuf r = {blob + off_end + a, b - a, 0, 0};
        uint32_t sl = rb_u32(&r);
        const uint8_t *sb = rb_take(&r, sl);
        if (r.err) { rc = ORC_ERR_FORMAT; break; }
        if ((rc = orc_rans_decode(sb, sl, nk, h->se_freqs, SE_ALPHABET, 1u << PAR_PREC_SE, se))) break;
        int64_t bstart[257];
        for (size_t i = 0; i < nk; i++) tmp[i] = se[i] & 0xFF;
        stable_order_by_exp(tmp, nk, order, bstart);
        uint32_t m = rb_u32(&r);
        const uint8_t *el = rb_take(&r, 2 * (size_t)m);
        if (r.err) { rc = ORC_ERR_FORMAT; break; }
        /* mant_sorted is np.empty: positions of buckets not listed stay
         * undefined in the reference; a valid stream lists every exponent. */
        for (size_t i = 0; i < nk; i++) ms[i] = 0;
        for (uint32_t q = 0; q < m; q++) {
            uint32_t e = get16(el + 2 * q);
            uint32_t cnt = rb_u32(&r), bl = rb_u32(&r);
            const uint8_t *mb = rb_take(&r, bl);
            if (r.err || e > 255) { rc = ORC_ERR_FORMAT; break; }
            size_t lo = (size_t)bstart[e], hi = (size_t)bstart[e + 1];
            /* mant_sorted[bstart[ev]:bstart[ev+1]] = bucket requires equal length */
            if ((size_t)cnt != hi - lo) { rc = ORC_ERR_FORMAT; break; }
            if ((rc = orc_rans_decode(mb, bl, cnt, h->mfreq[e], MANT_ALPHABET, 1u << PAR_PREC_M, ms + lo))) break;
        }
        if (rc) break;
        /* mant_slice[order] = mant_sorted; full[k::N] = ... (:557-561) */
        for (size_t j = 0; j < nk; j++) tmp[order[j]] = ms[j];
        for (size_t i = 0; i < nk; i++) {
            uint32_t s = se[i];
            out[k + i * N] = (uint16_t)((((s >> 8) & 1) << 15) | ((s & 0xFF) << 7) | (tmp[i] & 0xFFFF));
        }
    }
out:
    free(se); free(ms); free(tmp); free(order); free(h);
    return rc;
}

int orc_par1_decode(const uint8_t *blob, size_t len, size_t n_weights, uint16_t *out) {
    return orc_par1_decode_streams(blob, len, n_weights, out, 0, (size_t)-1);
}

/* ------------------------------------------------------------------------ */
/* bf16_se_tans  (bigsmall/codecs/bf16_tans.py + numba_rans.py)              */

/* bf16_tans.py:46-55 _encode_bucket: quantised freqs, nz idx, rANS stream. */
static int64_t tans_bucket(const int32_t *s, size_t n, int alphabet, uint32_t M, uint32_t *freqs,
                           uint8_t *out, size_t cap) {
    int64_t *cnt = (int64_t *)calloc(alphabet, sizeof(int64_t));
    if (!cnt) return ORC_ERR_ARG;
    for (size_t i = 0; i < n; i++) cnt[s[i]]++;
    int rc = orc_quantise_ref(cnt, alphabet, M, freqs);
    free(cnt);
    if (rc) return rc;
    return orc_rans_encode(s, n, freqs, alphabet, M, out, cap);
}

/* bf16_tans.py:68-118 encode */
int64_t orc_tans_encode(const uint16_t *w, size_t n, uint8_t *out, size_t cap) {
    if (n == 0) return 0;
    if (n > 0xFFFFFFFFull) return ORC_ERR_ARG;
    int32_t *sym = (int32_t *)malloc(sizeof(int32_t) * n);
    uint32_t *ex = (uint32_t *)malloc(sizeof(uint32_t) * n);
    size_t *order = (size_t *)malloc(sizeof(size_t) * n);
    uint8_t *cw = (uint8_t *)malloc(2 * n + 64);
    if (!sym || !ex || !order || !cw) { free(sym); free(ex); free(order); free(cw); return ORC_ERR_ARG; }
    int64_t rc = 0;
    wbuf wb = {out, 0, cap, 0};
    for (size_t i = 0; i < n; i++) { sym[i] = (int32_t)((w_sign(w[i]) << 8) | w_exp(w[i])); ex[i] = w_exp(w[i]); }
    uint32_t sf[SE_ALPHABET];
    int64_t sl = tans_bucket(sym, n, SE_ALPHABET, 4096, sf, cw, 2 * n + 64);
    if (sl < 0) { rc = sl; goto done; }
    int nnz = 0; for (int s = 0; s < SE_ALPHABET; s++) if (sf[s]) nnz++;
    wb_u32(&wb, (uint32_t)n); wb_u16(&wb, (uint32_t)nnz);
    for (int s = 0; s < SE_ALPHABET; s++) if (sf[s]) wb_u16(&wb, (uint32_t)s);
    for (int s = 0; s < SE_ALPHABET; s++) if (sf[s]) wb_u32(&wb, sf[s]);
    wb_u32(&wb, (uint32_t)sl); wb_put(&wb, cw, (size_t)sl);
    size_t mlen_pos = wb.len; wb_u32(&wb, 0);
    size_t mstart = wb.len;
    int64_t bstart[257];
    stable_order_by_exp(ex, n, order, bstart);
    int ne = 0; for (int e = 0; e < 256; e++) if (bstart[e + 1] > bstart[e]) ne++;
    wb_u32(&wb, (uint32_t)ne);
    for (int e = 0; e < 256; e++) if (bstart[e + 1] > bstart[e]) wb_u16(&wb, (uint32_t)e);
    for (int e = 0; e < 256 && !wb.err; e++) {
        size_t bc = (size_t)(bstart[e + 1] - bstart[e]);
        if (!bc) continue;
        for (size_t j = 0; j < bc; j++) sym[j] = (int32_t)w_mant(w[order[bstart[e] + j]]);
        uint32_t mf[MANT_ALPHABET];
        int64_t ml = tans_bucket(sym, bc, MANT_ALPHABET, 1024, mf, cw, 2 * n + 64);
        if (ml < 0) { rc = ml; goto done; }
        int k = 0; for (int m = 0; m < MANT_ALPHABET; m++) if (mf[m]) k++;
        wb_u32(&wb, (uint32_t)bc); wb_u8(&wb, (uint32_t)k);
        for (int m = 0; m < MANT_ALPHABET; m++) if (mf[m]) wb_u8(&wb, (uint32_t)m);
        for (int m = 0; m < MANT_ALPHABET; m++) if (mf[m]) wb_u32(&wb, mf[m]);
        wb_u32(&wb, (uint32_t)ml); wb_put(&wb, cw, (size_t)ml);
    }
    if (wb.err) { rc = ORC_ERR_CAP; goto done; }
    put32(out + mlen_pos, (uint32_t)(wb.len - mstart));
    rc = (int64_t)wb.len;
done:
    free(sym); free(ex); free(order); free(cw);
    return rc;
}

/* bf16_tans.py:121-167 decode (SE and buckets via numba_rans decode rules). */
int orc_tans_decode(const uint8_t *blob, size_t len, size_t n_weights, uint16_t *out) {
    if (n_weights == 0 || len == 0) return ORC_OK;
    rbuf r = {blob, len, 0, 0};
    uint32_t n = rb_u32(&r);
    if (r.err) return ORC_ERR_FORMAT;
    if (n != n_weights) return ORC_ERR_COUNT;
    if (n == 0) return ORC_OK;
    uint32_t nnz = rb_u16(&r);
    const uint8_t *idx = rb_take(&r, 2 * (size_t)nnz), *fq = rb_take(&r, 4 * (size_t)nnz);
    uint32_t cwl = rb_u32(&r);
    const uint8_t *cw = rb_take(&r, cwl);
    if (r.err) return ORC_ERR_FORMAT;
    uint32_t sf[SE_ALPHABET] = {0};
    for (uint32_t i = 0; i < nnz; i++) { uint32_t s = get16(idx + 2 * i); if (s >= SE_ALPHABET) return ORC_ERR_FORMAT; sf[s] = get32(fq + 4 * i); }
    uint32_t *se = (uint32_t *)malloc(sizeof(uint32_t) * n);
    uint32_t *ex = (uint32_t *)malloc(sizeof(uint32_t) * n);
    uint32_t *ms = (uint32_t *)calloc(n, sizeof(uint32_t));
    size_t *order = (size_t *)malloc(sizeof(size_t) * n);
    int rc = ORC_OK;
    if (!se || !ex || !ms || !order) { rc = ORC_ERR_ARG; goto out; }
    if ((rc = nb_decode_bytes(cw, cwl, n, sf, SE_ALPHABET, 12, se))) goto out;
    uint32_t mlen = rb_u32(&r);
    const uint8_t *mb = rb_take(&r, mlen);
    if (r.err) { rc = ORC_ERR_FORMAT; goto out; }
    rbuf m = {mb, mlen, 0, 0};
    uint32_t ne = rb_u32(&m);
    const uint8_t *el = rb_take(&m, 2 * (size_t)ne);
    if (m.err) { rc = ORC_ERR_FORMAT; goto out; }
    for (uint32_t i = 0; i < n; i++) ex[i] = se[i] & 0xFF;
    int64_t bstart[257];
    stable_order_by_exp(ex, n, order, bstart);
    for (uint32_t q = 0; q < ne; q++) {
        uint32_t e = get16(el + 2 * q);
        uint32_t nb = rb_u32(&m), k = rb_u8(&m);
        const uint8_t *mi = rb_take(&m, k), *mf = rb_take(&m, 4 * (size_t)k);
        uint32_t bl = rb_u32(&m);
        const uint8_t *bb = rb_take(&m, bl);
        if (m.err || e > 255) { rc = ORC_ERR_FORMAT; goto out; }
        uint32_t fr[MANT_ALPHABET] = {0};
        for (uint32_t j = 0; j < k; j++) { if (mi[j] >= MANT_ALPHABET) { rc = ORC_ERR_FORMAT; goto out; } fr[mi[j]] = get32(mf + 4 * j); }
        size_t lo = (size_t)bstart[e], hi = (size_t)bstart[e + 1];
        if ((size_t)nb != hi - lo) { rc = ORC_ERR_FORMAT; goto out; }
        if ((rc = nb_decode_bytes(bb, bl, nb, fr, MANT_ALPHABET, 10, ms + lo))) goto out;
    }
    /* mant[order_e] = mant_sorted (:332-336) */
    for (size_t j = 0; j < n; j++) ex[order[j]] = ms[j];
    for (size_t i = 0; i < n; i++)
        out[i] = (uint16_t)((((se[i] >> 8) & 1) << 15) | ((se[i] & 0xFF) << 7) | (ex[i] & 0xFFFF));
out:
    free(se); free(ex); free(ms); free(order);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* bf16_se_single_kernel  (bigsmall/codecs/single_kernel.py)                 */

/* single_kernel.py:121-156 _rans_encode_one (+ the caller's reversal): words
 * in decode order into `words`, returns count; *state = final state. */
static int64_t sk_encode_one(const int32_t *s, size_t n, const uint32_t *freqs, int alphabet,
                             uint32_t M, uint16_t *words, uint32_t *state_out) {
    if (n == 0) { *state_out = RANS_L; return 0; }
    uint32_t cum[SE_ALPHABET]; uint32_t c = 0;
    for (int i = 0; i < alphabet; i++) { cum[i] = c; c += freqs[i]; }
    uint64_t state = RANS_L, Lb = (1ull << 32) / M;
    size_t cnt = 0;
    for (size_t ii = n; ii-- > 0;) {
        uint64_t f = freqs[s[ii]], cf = cum[s[ii]];
        if (f == 0) return ORC_ERR_ARG;
        uint64_t upper = Lb * f;
        while (state >= upper) { words[cnt++] = (uint16_t)(state & 0xFFFF); state >>= 16; }
        state = (state / f) * M + cf + (state % f);
    }
    for (size_t i = 0; i < cnt / 2; i++) { uint16_t t = words[i]; words[i] = words[cnt - 1 - i]; words[cnt - 1 - i] = t; }
    *state_out = (uint32_t)state;
    return (int64_t)cnt;
}

/* single_kernel.py:193-428 _encode_full_kernel (layout :303-321). */
int64_t orc_sk_encode(const uint16_t *w, size_t n, uint8_t *out, size_t cap) {
    if (n == 0) return 0;
    if (n > 0xFFFFFFFFull) return ORC_ERR_ARG;
    int64_t se_cnt[SE_ALPHABET] = {0}, exp_cnt[256] = {0};
    int32_t *sym = (int32_t *)malloc(sizeof(int32_t) * n);
    uint8_t *ex = (uint8_t *)malloc(n);
    int32_t *ms = (int32_t *)malloc(sizeof(int32_t) * n);
    uint16_t *wr = (uint16_t *)malloc(sizeof(uint16_t) * (n + 8));
    if (!sym || !ex || !ms || !wr) { free(sym); free(ex); free(ms); free(wr); return ORC_ERR_ARG; }
    for (size_t i = 0; i < n; i++) {
        sym[i] = (int32_t)((w_sign(w[i]) << 8) | w_exp(w[i])); ex[i] = (uint8_t)w_exp(w[i]);
        se_cnt[sym[i]]++; exp_cnt[ex[i]]++;
    }
    uint32_t sf[SE_ALPHABET];
    orc_quantise_sk(se_cnt, SE_ALPHABET, 4096, sf);
    int64_t bstart[257]; bstart[0] = 0;
    for (int e = 0; e < 256; e++) bstart[e + 1] = bstart[e] + exp_cnt[e];
    int64_t cur[256]; for (int e = 0; e < 256; e++) cur[e] = bstart[e];
    for (size_t i = 0; i < n; i++) ms[cur[ex[i]]++] = (int32_t)w_mant(w[i]);   /* :229-241 */
    wbuf wb = {out, 0, cap, 0};
    int64_t rc = 0;
    uint32_t st;
    int64_t nw = sk_encode_one(sym, n, sf, SE_ALPHABET, 4096, wr, &st);
    if (nw < 0) { rc = nw; goto done; }
    int nnz = 0; for (int s = 0; s < SE_ALPHABET; s++) if (sf[s] > 0) nnz++;
    wb_u32(&wb, (uint32_t)n); wb_u16(&wb, (uint32_t)nnz);
    for (int s = 0; s < SE_ALPHABET; s++) if (sf[s] > 0) wb_u16(&wb, (uint32_t)s);
    for (int s = 0; s < SE_ALPHABET; s++) if (sf[s] > 0) wb_u32(&wb, sf[s]);
    wb_u32(&wb, st); wb_u32(&wb, (uint32_t)nw);
    for (int64_t i = 0; i < nw; i++) wb_u16(&wb, wr[i]);
    int ne = 0; for (int e = 0; e < 256; e++) if (exp_cnt[e]) ne++;
    wb_u32(&wb, (uint32_t)ne);
    for (int e = 0; e < 256 && !wb.err; e++) {
        if (!exp_cnt[e]) continue;
        int64_t bc[MANT_ALPHABET] = {0};
        for (int64_t i = bstart[e]; i < bstart[e + 1]; i++) bc[ms[i]]++;
        uint32_t mf[MANT_ALPHABET];
        orc_quantise_sk(bc, MANT_ALPHABET, 1024, mf);
        uint32_t mst;
        int64_t mw = sk_encode_one(ms + bstart[e], (size_t)(bstart[e + 1] - bstart[e]), mf, MANT_ALPHABET, 1024, wr, &mst);
        if (mw < 0) { rc = mw; goto done; }
        wb_u16(&wb, (uint32_t)e);
        int k = 0; for (int m = 0; m < MANT_ALPHABET; m++) if (mf[m] > 0) k++;
        wb_u8(&wb, (uint32_t)k);
        for (int m = 0; m < MANT_ALPHABET; m++) if (mf[m] > 0) wb_u8(&wb, (uint32_t)m);
        for (int m = 0; m < MANT_ALPHABET; m++) if (mf[m] > 0) wb_u32(&wb, mf[m]);
        wb_u32(&wb, mst); wb_u32(&wb, (uint32_t)(bstart[e + 1] - bstart[e])); wb_u32(&wb, (uint32_t)mw);
        for (int64_t i = 0; i < mw; i++) wb_u16(&wb, wr[i]);
    }
    rc = wb.err ? ORC_ERR_CAP : (int64_t)wb.len;
done:
    free(sym); free(ex); free(ms); free(wr);
    return rc;
}

/* single_kernel.py:431-580 _decode_full_kernel (uint32 arithmetic, renorm while
 * state < L and pos < end; un-sort by cursor walk). */
int orc_sk_decode(const uint8_t *blob, size_t len, size_t n_weights, uint16_t *out) {
    if (n_weights == 0 || len == 0) return ORC_OK;          /* :605-606 */
    rbuf r = {blob, len, 0, 0};
    uint32_t n = rb_u32(&r);
    if (r.err) return ORC_ERR_FORMAT;
    if (n != n_weights) return ORC_ERR_COUNT;               /* :445-446 */
    uint32_t nnz = rb_u16(&r);
    const uint8_t *idx = rb_take(&r, 2 * (size_t)nnz), *fq = rb_take(&r, 4 * (size_t)nnz);
    uint32_t st = rb_u32(&r), nc = rb_u32(&r);
    const uint8_t *wd = rb_take(&r, 2 * (size_t)nc);
    if (r.err) return ORC_ERR_FORMAT;
    uint32_t sf[SE_ALPHABET] = {0}, cum[SE_ALPHABET];
    for (uint32_t i = 0; i < nnz; i++) { uint32_t s = get16(idx + 2 * i); if (s >= SE_ALPHABET) return ORC_ERR_FORMAT; sf[s] = get32(fq + 4 * i); }
    uint32_t c = 0; for (int i = 0; i < SE_ALPHABET; i++) { cum[i] = c; c += sf[i]; }
    uint32_t *tbl = (uint32_t *)calloc(4096, sizeof(uint32_t));
    uint16_t *d = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)nc + 2));
    uint32_t *se = (uint32_t *)malloc(sizeof(uint32_t) * ((size_t)n + 1));
    uint8_t *msort = (uint8_t *)calloc((size_t)n + 1, 1);
    uint32_t *tmp = (uint32_t *)malloc(sizeof(uint32_t) * ((size_t)n + 1));
    int rc = ORC_OK;
    if (!tbl || !d || !se || !msort || !tmp) { rc = ORC_ERR_ARG; goto out; }
    for (int s = 0; s < SE_ALPHABET; s++)
        for (uint32_t k = 0; k < sf[s] && cum[s] + k < 4096; k++) tbl[cum[s] + k] = (uint32_t)s;
    d[0] = (uint16_t)(st & 0xFFFF); d[1] = (uint16_t)(st >> 16);
    for (uint32_t i = 0; i < nc; i++) d[2 + i] = (uint16_t)get16(wd + 2 * i);
    nb_decode_u16(d, (size_t)nc + 2, n, sf, cum, tbl, 12, se);
    int64_t ecnt[256] = {0}, bstart[257];
    for (uint32_t i = 0; i < n; i++) ecnt[se[i] & 0xFF]++;
    bstart[0] = 0; for (int e = 0; e < 256; e++) bstart[e + 1] = bstart[e] + ecnt[e];
    uint32_t ne = rb_u32(&r);
    for (uint32_t b = 0; b < ne && !r.err; b++) {
        uint32_t e = rb_u16(&r), k = rb_u8(&r);
        const uint8_t *mi = rb_take(&r, k), *mf = rb_take(&r, 4 * (size_t)k);
        uint32_t mst = rb_u32(&r), bsz = rb_u32(&r), mnc = rb_u32(&r);
        const uint8_t *mw = rb_take(&r, 2 * (size_t)mnc);
        if (r.err || e > 255) { rc = ORC_ERR_FORMAT; goto out; }
        uint32_t fr[MANT_ALPHABET] = {0}, mcum[MANT_ALPHABET], mt[1024];
        for (uint32_t j = 0; j < k; j++) { if (mi[j] >= MANT_ALPHABET) { rc = ORC_ERR_FORMAT; goto out; } fr[mi[j]] = get32(mf + 4 * j); }
        uint32_t cc = 0; for (int i = 0; i < MANT_ALPHABET; i++) { mcum[i] = cc; cc += fr[i]; }
        memset(mt, 0, sizeof(mt));
        for (int s = 0; s < MANT_ALPHABET; s++)
            for (uint32_t q = 0; q < fr[s] && mcum[s] + q < 1024; q++) mt[mcum[s] + q] = (uint32_t)s;
        if ((int64_t)bstart[e] + bsz > (int64_t)n) { rc = ORC_ERR_FORMAT; goto out; }
        uint16_t *md = (uint16_t *)malloc(sizeof(uint16_t) * ((size_t)mnc + 2));
        if (!md) { rc = ORC_ERR_ARG; goto out; }
        md[0] = (uint16_t)(mst & 0xFFFF); md[1] = (uint16_t)(mst >> 16);
        for (uint32_t i = 0; i < mnc; i++) md[2 + i] = (uint16_t)get16(mw + 2 * i);
        nb_decode_u16(md, (size_t)mnc + 2, bsz, fr, mcum, mt, 10, tmp);
        for (uint32_t i = 0; i < bsz; i++) msort[bstart[e] + i] = (uint8_t)tmp[i];
        free(md);
    }
    if (r.err) { rc = ORC_ERR_FORMAT; goto out; }
    {
        int64_t cur[256]; for (int e = 0; e < 256; e++) cur[e] = bstart[e];
        for (uint32_t i = 0; i < n; i++) {                   /* :570-580 */
            uint32_t e = se[i] & 0xFF;
            uint32_t m = msort[cur[e]++];
            out[i] = (uint16_t)((((se[i] >> 8) & 1) << 15) | (e << 7) | m);
        }
    }
out:
    free(tbl); free(d); free(se); free(msort); free(tmp);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* BSCK — the engine's GPU-native chunked container format (no reference
 * counterpart). CPU restatement of the device decoder's semantics: the oracle
 * for the product encoder and the GPU decoder. Format:
 *   [0]  "BSCK"  [4] u8 version (2 or 3)  [5] u8 elem_bytes (1|2)  [6] u8 plane_mode
 *   [7]  u8 prec_log2 (12)  [8] u64 n  [16] u32 steps  [20] u16 lanes (64*K, K in 1,2,4)
 *   [22] u16 n_syms  [24] u32 n_chunks  [28] u8 coder (0 rANS; version 3: 1 tANS with a
 *        state array, 2 tANS with the states at the stream head), 3 zero bytes
 *   [32] n_syms x u32 symbol entries: bits 0..15 value, bits 16..28 freq,
 *        bit 31 = consumes one plane byte
 *   pad to 16; tANS only: 4096 x u32 decode table {newX:12, nb:4, symbol:8, 0:8}
 *   n_chunks x {u64 offset, u32 n_words (rANS) or n_bits (tANS), u32 n_plane}
 *   version 3, plane modes 1 and 3: pad to 256, the full chunks' dense planes (nf*lanes*steps bytes)
 *   chunk: lanes x u32 initial states (not in coder 2) | rANS: n_words x u16,
 *          tANS: ceil(n_bits/32) x u32, padded to 16 | n_plane bytes (pad 16),
 *          the plane omitted for a full chunk of a version-3 blob in plane
 *          modes 1 and 3
 *   version 3: pad to 256 (blob lengths are multiples of 256); coder 2: the
 *   blob holds 256 bytes from every chunk's offset
 * Elements: bf16 words, or bytes; in plane mode 3 (fp8 exponent pairs) an
 * element is a pair of bytes (a 16-bit word) and n counts bytes. With
 * per = lanes*steps and nf = ne / per full chunks (ne = coded elements),
 * element j of full chunk c sits at ((j / 512) * nf + c) * 512 + j % 512 in
 * version 3 (512-element units interleaved across the full chunks) and at
 * c*per + j in version 2; element j of the partial chunk (c = nf) at
 * nf*per + j. With K = lanes/64, state v = g*64 + l (wavefront lane l,
 * group g) decodes element t*lanes + l*K + g at step t.
 * rANS (coder 0; bigsmall/codecs/rans.py:165-207's state machine, M = 4096,
 * L = 2^16): slot = x & 4095; x = f[s]*(x >> 12) + slot - cum[s]; if x < L,
 * x = x << 16 | the next word; words are consumed per step in ascending v
 * order among states that fell below L. A chunk ends with every x == L.
 * tANS (coders 1 and 2): X in [0, 4096); entry = table[X]; s = its symbol;
 * X = newX + the next nb bits of the chunk's LSB-first bit stream, read in
 * chunk element order (per step, lanes ascending, a lane's states ascending);
 * in plane mode 2 a consuming symbol then reads its 8 plane bits. A chunk
 * ends with every X == 0 and every bit read. Coder 2's stream starts with the
 * initial states, 12 bits each, in the same reading order (lane l's state g at
 * bit 12*(l*K + g)); coder 1 keeps them in the u32 array.
 * Plane bytes: plane_mode 1/3 (dense): every element has one, stored in blocks
 * of B steps (B = 8 for K <= 2, 4 for K = 4); the byte of state (g, l) for step
 * B*b+q sits at byte l*B*K + q*K + g of the chunk's plane block b (B*lanes
 * bytes), which is block b*nf + c of the plane region for a full chunk of a
 * version-3 blob, and at b*B*lanes of the inline plane otherwise.
 * plane_mode 2 (compact): consuming elements read bytes in decode order (rANS)
 * or from the stream (tANS).
 * bf16 value = symbol value | plane byte's bit 7 << 15 | its bits 0..6.
 * Pair value (mode 3): symbol value k = e0 | e1 << 4, plane byte p =
 * m0 | s1 << 3 | m1 << 4 | s0 << 7: byte 0 = s0 << 7 | e0 << 3 | m0,
 * byte 1 = s1 << 7 | e1 << 3 | m1.
 * ------------------------------------------------------------------------ */

/* LSB-first bit reader over a whole-u32-word stream */
typedef struct { const uint8_t *p; uint64_t nbits, pos; } bitrd;
static uint32_t br_take(bitrd *b, uint32_t k, int *err) {
    uint32_t v = 0;
    for (uint32_t i = 0; i < k; i++, b->pos++) {
        if (b->pos >= b->nbits) { *err = 1; return 0; }
        v |= (uint32_t)((b->p[b->pos >> 3] >> (b->pos & 7)) & 1u) << i;
    }
    return v;
}

/* The tANS decode table of quantised frequencies (sum 4096), built the
 * long way: the slots of symbol s, [cum_s, cum_s + f_s), are placed at
 * position slot * 2563 mod 4096; scanning positions upwards, the k-th
 * position of s gets next = f_s + k, nb = the shift that brings next into
 * [4096, 8192), newX = next << nb minus 4096. */
int orc_tans_table(const uint32_t *freq, int nsym, uint32_t *out) {
    if (nsym < 1 || nsym > 256) return ORC_ERR_ARG;
    uint32_t cum = 0, at[4096], seen[256] = {0};
    for (int s = 0; s < nsym; s++) {
        if (freq[s] == 0) return ORC_ERR_ARG;
        for (uint32_t k = 0; k < freq[s]; k++) {
            if (cum + k >= 4096) return ORC_ERR_ARG;
            at[((cum + k) * 2563u) % 4096u] = (uint32_t)s;
        }
        cum += freq[s];
    }
    if (cum != 4096) return ORC_ERR_ARG;
    for (uint32_t p = 0; p < 4096; p++) {
        uint32_t s = at[p], next = freq[s] + seen[s]++, nb = 0;
        while ((next << nb) < 4096u) nb++;
        out[p] = ((next << nb) - 4096u) | (nb << 12) | (s << 16);
    }
    return ORC_OK;
}

/* Chunks [c0, c1) (clamped to the blob's count): each writes only its own
 * elements, so disjoint ranges may run on separate threads. */
int orc_chunk_decode_range(const uint8_t *blob, size_t len, size_t n_weights, void *out_v, size_t c0, size_t c1) {
    if (len < 32 || memcmp(blob, "BSCK", 4) != 0) return ORC_ERR_FORMAT;
    uint32_t ver = blob[4], eb = blob[5], mode = blob[6], prec = blob[7];
    uint64_t n = get64(blob + 8);
    uint32_t steps = get32(blob + 16), lanes = get16(blob + 20), nsym = get16(blob + 22), nch = get32(blob + 24);
    uint32_t coder = blob[28];
    if ((ver != 2 && ver != 3) || (eb != 1 && eb != 2) || mode > 3 || prec != 12 ||
        (lanes != 64 && lanes != 128 && lanes != 256) || steps == 0 || steps % 16 || coder > 2 ||
        blob[29] || blob[30] || blob[31] || (ver == 2 && coder != 0) ||
        (eb == 1 && mode != 0 && mode != 3) || (eb == 2 && mode == 3) || (mode == 3 && ver != 3))
        return ORC_ERR_FORMAT;
    if (n != n_weights) return ORC_ERR_COUNT;
    if (mode == 3 && n % 2) return ORC_ERR_FORMAT;
    if (nsym == 0 || nsym > 256) return ORC_ERR_FORMAT;
    uint64_t ne = mode == 3 ? n / 2 : n;                     /* coded elements */
    uint64_t per = (uint64_t)lanes * steps;
    if (nch != (ne + per - 1) / per) return ORC_ERR_FORMAT;
    size_t stab = (32 + 4 * (size_t)nsym + 15) & ~(size_t)15;
    size_t ctab = stab + (coder ? 4096 * 4 : 0);
    if (ctab + 16 * (size_t)nch > len) return ORC_ERR_FORMAT;
    uint64_t nf = ne / per;                                  /* full chunks */
    int region = ver == 3 && (mode == 1 || mode == 3);       /* full chunks' planes in the plane region */
    size_t preg = (ctab + 16 * (size_t)nch + 255) & ~(size_t)255;
    if (region && preg + nf * per > len) return ORC_ERR_FORMAT;
    uint32_t val[256], fr[256], cons[256], cum[256], c = 0;
    for (uint32_t s = 0; s < nsym; s++) {
        uint32_t e = get32(blob + 32 + 4 * s);
        val[s] = e & 0xFFFF; fr[s] = (e >> 16) & 0x1FFF; cons[s] = e >> 31;
        if (fr[s] == 0) return ORC_ERR_FORMAT;
        cum[s] = c; c += fr[s];
    }
    if (c != 4096) return ORC_ERR_FORMAT;
    uint8_t slot2sym[4096];
    uint32_t ttab[4096];
    if (coder == 0) {
        for (uint32_t s = 0; s < nsym; s++) for (uint32_t k = 0; k < fr[s]; k++) slot2sym[cum[s] + k] = (uint8_t)s;
    } else {
        for (uint32_t p = 0; p < 4096; p++) {
            uint32_t e = get32(blob + stab + 4 * p), nb = (e >> 12) & 15, s = (e >> 16) & 0xFF;
            if ((e >> 24) || s >= nsym || nb > 12 || (e & 0xFFF) + (1u << nb) > 4096) return ORC_ERR_FORMAT;
            ttab[p] = e;
        }
    }
    const uint32_t K = lanes / 64, bs = lanes == 256 ? 4 : 8;   /* states per lane, steps per plane block */
    if (c1 > nch) c1 = nch;
    for (size_t ci = c0; ci < c1; ci++) {
        const uint8_t *ce = blob + ctab + 16 * (size_t)ci;
        uint64_t off = get64(ce); uint32_t nw = get32(ce + 8), np = get32(ce + 12);
        int split = region && ci < nf;
        size_t sbytes = coder == 0 ? ((size_t)nw * 2 + 15) & ~(size_t)15
                                   : ((((size_t)nw + 31) / 32) * 4 + 15) & ~(size_t)15;
        size_t pbytes = split ? 0 : ((size_t)np + 15) & ~(size_t)15;
        size_t sarr = coder == 2 ? 0 : 4 * (size_t)lanes;          /* the u32 state array */
        if (off % 16 || off + sarr + sbytes + pbytes > len || (coder == 2 && off + 256 > len)) return ORC_ERR_FORMAT;
        const uint8_t *st = blob + off, *wd = st + sarr, *pl = wd + sbytes;
        uint64_t nc = ci < nf ? per : ne - nf * per;
        uint64_t nsteps = (nc + lanes - 1) / lanes;
        uint32_t x[256];
        uint64_t wp = 0, pp = 0;
        bitrd br = {wd, nw, 0};
        int err = 0;
        if (coder == 2) {
            for (uint32_t i = 0; i < lanes; i++) x[(i % K) * 64 + i / K] = br_take(&br, 12, &err);
            if (err) return ORC_ERR_FORMAT;
        } else {
            for (uint32_t l = 0; l < lanes; l++) x[l] = get32(st + 4 * l);
        }
        if (coder == 1) for (uint32_t l = 0; l < lanes; l++) if (x[l] >= 4096) return ORC_ERR_FORMAT;
        for (uint64_t t = 0; t < nsteps; t++) {
            for (uint32_t i = 0; i < lanes; i++) {
                /* rANS: states in v order (group-major); tANS: chunk element order (lane-major) */
                uint32_t g = coder == 0 ? i / 64 : i % K, wl = coder == 0 ? i % 64 : i / K, sv = g * 64 + wl;
                uint64_t j = t * lanes + (uint64_t)wl * K + g;
                if (j >= nc) continue;
                uint32_t s;
                if (coder == 0) {
                    uint32_t slot = x[sv] & 4095;
                    s = slot2sym[slot];
                    x[sv] = fr[s] * (x[sv] >> 12) + slot - cum[s];
                    if (x[sv] < RANS_L) {
                        if (wp >= nw) return ORC_ERR_FORMAT;
                        x[sv] = (x[sv] << 16) | get16(wd + 2 * wp); wp++;
                    }
                } else {
                    uint32_t e = ttab[x[sv]];
                    s = (e >> 16) & 0xFF;
                    x[sv] = (e & 0xFFF) + br_take(&br, (e >> 12) & 15, &err);
                }
                uint32_t v = val[s];
                if (cons[s]) {
                    uint32_t b;
                    if (mode == 1 || mode == 3) {
                        uint64_t blk = t / bs, q = t % bs;
                        uint64_t in_blk = (uint64_t)wl * bs * K + q * K + g;
                        if (blk * bs * lanes + in_blk >= np) return ORC_ERR_FORMAT;
                        b = split ? blob[preg + (blk * nf + ci) * bs * lanes + in_blk] : pl[blk * bs * lanes + in_blk];
                    } else if (mode == 2 && coder == 0) {
                        if (pp >= np) return ORC_ERR_FORMAT;
                        b = pl[pp++];
                    } else if (mode == 2) {
                        b = br_take(&br, 8, &err);
                    } else return ORC_ERR_FORMAT;
                    if (mode == 3) {
                        uint32_t e0 = v & 15, e1 = (v >> 4) & 15;
                        uint32_t b0 = (b & 0x80) | (e0 << 3) | (b & 7);
                        uint32_t b1 = (((b >> 3) & 1) << 7) | (e1 << 3) | ((b >> 4) & 7);
                        v = b0 | (b1 << 8);
                    } else {
                        v = v | (b & 0x7F) | ((b & 0x80) << 8);
                    }
                }
                if (err) return ORC_ERR_FORMAT;
                uint64_t e = ci < nf && ver == 3 ? ((j / 512) * nf + ci) * 512 + j % 512 : (uint64_t)ci * per + j;
                if (eb == 2 || mode == 3) ((uint16_t *)out_v)[e] = (uint16_t)v;
                else ((uint8_t *)out_v)[e] = (uint8_t)v;
            }
        }
        for (uint32_t l = 0; l < lanes; l++) if (x[l] != (coder == 0 ? RANS_L : 0)) return ORC_ERR_FORMAT;
        if (coder == 0 && wp != nw) return ORC_ERR_FORMAT;
        if (coder != 0 && br.pos != nw) return ORC_ERR_FORMAT;
        if (coder == 0 && mode == 2 && pp != np) return ORC_ERR_FORMAT;
    }
    return ORC_OK;
}

int orc_chunk_decode(const uint8_t *blob, size_t len, size_t n_weights, void *out_v) {
    return orc_chunk_decode_range(blob, len, n_weights, out_v, 0, (size_t)-1);
}
