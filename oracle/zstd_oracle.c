/*
 * zstd_oracle.c -- CPU restatement of Zstandard frame decoding.
 *
 * TEST INFRASTRUCTURE ONLY (see ptwm_oracle.h).
 *
 * The reference's Zstd plane codec (crates/ptwm-core/src/codecs/zstd.rs,
 * codec_tagged.rs:198-307) hands the payload to the `zstd` crate 0.13.3
 * (zstd-sys 2.0.16+zstd.1.5.7, Cargo.lock), a binding of libzstd, whose
 * decode_all / stream decoder reads one or more concatenated frames.  The
 * crate is a third-party dependency absent from the reference tree; this
 * file restates the published format, RFC 8878 ("Zstandard Compression and
 * the application/zstd Media Type"), section by section:
 *   3.1.1      frames: magic, frame header, blocks, content checksum
 *   3.1.2      skippable frames
 *   3.1.1.2    blocks: raw, RLE, compressed (Block_Maximum_Size 128 KiB)
 *   3.1.1.3.1  literals section (raw, RLE, Huffman 1 or 4 streams, treeless)
 *   3.1.1.3.2  sequences section (predefined / RLE / FSE / repeat tables)
 *   3.1.1.4    sequence execution and repeat offsets
 *   4.1        FSE table description and decoding tables
 *   4.2        Huffman tree description (direct or FSE-coded weights)
 * with libzstd's decoder limits where the RFC leaves a choice: window sizes
 * above 2^27 + 1 bytes are refused (ZSTD_MAXWINDOWSIZE_DEFAULT of the
 * streaming decoder), and a frame with a dictionary id is refused (the
 * plane codec loads no dictionary).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "ptwm_oracle.h"

#define ZBLOCK_MAX (128u * 1024u)

static uint32_t zld32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
static int zhighbit(uint32_t x) { return 31 - __builtin_clz(x); }

/* ---- forward bit reader (FSE table descriptions, 4.1.1) ---- */
typedef struct { const uint8_t *p; size_t n; uint64_t bit; } fwd_t;
static uint32_t fwd_peek(const fwd_t *r, int nb) {
    uint32_t v = 0;
    for (int i = 0; i < nb; i++) {
        uint64_t b = r->bit + (uint64_t)i;
        uint32_t bitv = (b >> 3) < r->n ? (r->p[b >> 3] >> (b & 7)) & 1u : 0u;
        v |= bitv << i;
    }
    return v;
}

/* ---- backward bit reader (Huffman streams, FSE bitstreams, 4.1 / 4.2.2):
 * the stream is read from its last byte toward its first, most significant
 * bit first; the last byte's highest set bit is a start marker.  `avail`
 * counts the real bits; a read past them returns zeros and `used` keeps
 * counting, which is how the Huffman-weight loop notices its end. */
typedef struct { const uint8_t *p; int64_t avail; int64_t used; } bwd_t;
static int bwd_init(bwd_t *r, const uint8_t *p, size_t n) {
    if (n == 0 || p[n - 1] == 0) return -1;
    r->p = p;
    r->avail = (int64_t)n * 8 - (8 - zhighbit(p[n - 1]));
    r->used = 0;
    return 0;
}
static uint32_t bwd_peek(const bwd_t *r, int nb) {
    uint32_t v = 0;
    for (int i = 0; i < nb; i++) {
        int64_t b = r->avail - 1 - r->used - i;   /* bit index from the stream's start */
        uint32_t bitv = b >= 0 ? (r->p[b >> 3] >> (b & 7)) & 1u : 0u;
        v = (v << 1) | bitv;
    }
    return v;
}
static uint32_t bwd_read(bwd_t *r, int nb) { uint32_t v = bwd_peek(r, nb); r->used += nb; return v; }

/* ---- FSE (4.1) ---- */
typedef struct { uint8_t sym; uint8_t nb; uint16_t base; } fse_e;
typedef struct { int al; fse_e t[512]; } fse_t;

/* 4.1.1: normalized counts; returns bytes consumed or -1 */
static int64_t fse_read_ncount(const uint8_t *p, size_t n, int max_al, int max_sym, int16_t *norm, int *al_out, int *nsym) {
    if (n < 1) return -1;
    fwd_t r = {p, n, 0};
    int al = (int)fwd_peek(&r, 4) + 5;
    r.bit = 4;
    if (al > max_al) return -1;
    int remaining = (1 << al) + 1, threshold = 1 << al, nb = al + 1, s = 0;
    int prev0 = 0;
    while (remaining > 1 && s <= max_sym) {
        if (prev0) {
            int n0 = s;
            for (;;) {
                if ((r.bit + 2 + 7) / 8 > n) return -1;
                uint32_t rep = fwd_peek(&r, 2);
                r.bit += 2;
                n0 += (int)rep;
                if (rep != 3) break;
            }
            if (n0 > max_sym) return -1;
            while (s < n0) norm[s++] = 0;
            if (s > max_sym) break;   /* libzstd: loop test on charnum */
        }
        int mx = (2 * threshold - 1) - remaining;
        int count;
        uint32_t low = fwd_peek(&r, nb - 1);
        if ((int)low < mx) {
            count = (int)low;
            r.bit += (uint64_t)(nb - 1);
        } else {
            count = (int)fwd_peek(&r, nb);
            if (count >= threshold) count -= mx;
            r.bit += (uint64_t)nb;
        }
        if ((r.bit + 7) / 8 > n) return -1;
        count--;
        remaining -= count < 0 ? -count : count;
        norm[s++] = (int16_t)count;
        prev0 = count == 0;
        while (remaining < threshold) { nb--; threshold >>= 1; }
    }
    if (remaining != 1) return -1;
    for (int k = s; k <= max_sym; k++) norm[k] = 0;
    *al_out = al;
    *nsym = s;
    return (int64_t)((r.bit + 7) / 8);
}

/* 4.1.1 decoding table: -1 ("less than 1") symbols at the top, the rest
 * spread with step (size/2 + size/8 + 3), skipping the top slots */
static int fse_build(fse_t *f, const int16_t *norm, int nsym, int al) {
    uint32_t size = 1u << al, high = size - 1, next[256];
    f->al = al;
    for (int s = 0; s < nsym; s++) {
        if (norm[s] == -1) { f->t[high--].sym = (uint8_t)s; next[s] = 1; }
        else next[s] = (uint32_t)norm[s];
    }
    uint32_t pos = 0, step = (size >> 1) + (size >> 3) + 3, mask = size - 1;
    for (int s = 0; s < nsym; s++) {
        for (int i = 0; i < norm[s]; i++) {
            f->t[pos].sym = (uint8_t)s;
            do { pos = (pos + step) & mask; } while (pos > high);
        }
    }
    if (pos != 0) return -1;
    for (uint32_t u = 0; u < size; u++) {
        uint32_t s = f->t[u].sym, x = next[s]++;
        int nbits = al - zhighbit(x);
        f->t[u].nb = (uint8_t)nbits;
        f->t[u].base = (uint16_t)((x << nbits) - size);
    }
    return 0;
}

static void fse_rle(fse_t *f, uint8_t sym) { f->al = 0; f->t[0].sym = sym; f->t[0].nb = 0; f->t[0].base = 0; }

/* ---- Huffman (4.2) ---- */
typedef struct { int max_bits; uint8_t sym[4096]; uint8_t nb[4096]; } huf_t;

static int huf_from_weights(huf_t *h, const uint8_t *w, int nw) {
    /* the last weight is implied: the total 2^(w-1) rounds up to a power of 2 */
    uint32_t total = 0;
    for (int i = 0; i < nw; i++) {
        if (w[i] > 12) return -1;   /* HUF_TABLELOG_MAX of libzstd */
        if (w[i]) total += 1u << (w[i] - 1);
    }
    if (total == 0) return -1;
    int max_bits = zhighbit(total) + 1;
    uint32_t rest = (1u << max_bits) - total;
    if (rest & (rest - 1)) return -1;
    int last_w = zhighbit(rest) + 1;
    if (max_bits > 12 || nw + 1 > 256) return -1;
    uint8_t ww[256] = {0};
    memcpy(ww, w, (size_t)nw);
    ww[nw] = (uint8_t)last_w;
    int ns = nw + 1;
    /* codes in order of increasing weight, then symbol: each symbol of
     * weight k fills 2^(k-1) consecutive slots */
    uint32_t rank[13] = {0}, start = 0;
    for (int i = 0; i < ns; i++) rank[ww[i]]++;
    if (rank[1] < 2 || (rank[1] & 1)) return -1;   /* weight 1: at least two, an even count */
    uint32_t pos[13];
    for (int k = 1; k <= 12; k++) { pos[k] = start; start += rank[k] << (k - 1); }
    if (start != (1u << max_bits)) return -1;
    h->max_bits = max_bits;
    for (int i = 0; i < ns; i++) {
        int k = ww[i];
        if (!k) continue;
        uint32_t len = 1u << (k - 1);
        for (uint32_t j = 0; j < len; j++) {
            h->sym[pos[k] + j] = (uint8_t)i;
            h->nb[pos[k] + j] = (uint8_t)(max_bits + 1 - k);
        }
        pos[k] += len;
    }
    return 0;
}

/* 4.2.1: tree description; returns bytes consumed or -1 */
static int64_t huf_read_tree(huf_t *h, const uint8_t *p, size_t n) {
    if (n < 1) return -1;
    uint8_t w[256];
    int nw = 0;
    size_t hb = p[0];
    if (hb >= 128) {
        nw = (int)hb - 127;
        size_t bytes = ((size_t)nw + 1) / 2;
        if (1 + bytes > n) return -1;
        for (int i = 0; i < nw; i++) {
            uint8_t b = p[1 + i / 2];
            w[i] = (i % 2 == 0) ? (uint8_t)(b >> 4) : (uint8_t)(b & 15);
        }
        if (huf_from_weights(h, w, nw)) return -1;
        return (int64_t)(1 + bytes);
    }
    if (1 + hb > n) return -1;
    /* FSE-coded weights: a table of accuracy <= 6, two interleaved states */
    const uint8_t *q = p + 1;
    int16_t norm[256];
    int al, nsym;
    int64_t used = fse_read_ncount(q, hb, 6, 255, norm, &al, &nsym);
    if (used < 0 || (size_t)used > hb) return -1;
    fse_t *f = (fse_t *)malloc(sizeof(fse_t));
    if (!f) return -1;
    if (fse_build(f, norm, nsym, al)) { free(f); return -1; }
    bwd_t r;
    if (bwd_init(&r, q + used, hb - (size_t)used)) { free(f); return -1; }
    uint32_t s1 = bwd_read(&r, al), s2 = bwd_read(&r, al);
    for (;;) {
        if (nw > 253) { free(f); return -1; }
        w[nw++] = f->t[s1].sym;
        s1 = f->t[s1].base + bwd_read(&r, f->t[s1].nb);
        if (r.used > r.avail) { w[nw++] = f->t[s2].sym; break; }
        if (nw > 253) { free(f); return -1; }
        w[nw++] = f->t[s2].sym;
        s2 = f->t[s2].base + bwd_read(&r, f->t[s2].nb);
        if (r.used > r.avail) { w[nw++] = f->t[s1].sym; break; }
    }
    free(f);
    if (huf_from_weights(h, w, nw)) return -1;
    return (int64_t)(1 + hb);
}

static int huf_stream(const huf_t *h, const uint8_t *p, size_t n, uint8_t *out, size_t cnt) {
    bwd_t r;
    if (bwd_init(&r, p, n)) return -1;
    for (size_t i = 0; i < cnt; i++) {
        uint32_t v = bwd_peek(&r, h->max_bits);
        out[i] = h->sym[v];
        r.used += h->nb[v];
    }
    return r.used == r.avail ? 0 : -1;   /* the stream is consumed exactly */
}

/* ---- sequence code tables (3.1.1.3.2.1) ---- */
static const uint32_t LL_BASE[36] = {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 18, 20, 22, 24, 28, 32, 40,
                                     48, 64, 128, 256, 512, 1024, 2048, 4096, 8192, 16384, 32768, 65536};
static const uint8_t LL_BITS[36] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 2, 2, 3, 3,
                                    4, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16};
static const uint32_t ML_BASE[53] = {3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20,
                                     21, 22, 23, 24, 25, 26, 27, 28, 29, 30, 31, 32, 33, 34, 35, 37, 39, 41,
                                     43, 47, 51, 59, 67, 83, 99, 131, 259, 515, 1027, 2051, 4099, 8195, 16387, 32771,
                                     65539};
static const uint8_t ML_BITS[53] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0,
                                    0, 0, 0, 0, 0, 1, 1, 1, 1, 2, 2, 3, 3, 4, 4, 5, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16};
/* default distributions (3.1.1.3.2.2) */
static const int16_t LL_DEF[36] = {4, 3, 2, 2, 2, 2, 2, 2, 2, 2, 2, 2, 2, 1, 1, 1, 2, 2, 2, 2, 2, 2, 2, 2,
                                   2, 3, 2, 1, 1, 1, 1, 1, -1, -1, -1, -1};
static const int16_t ML_DEF[53] = {1, 4, 3, 2, 2, 2, 2, 2, 2, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1,
                                   1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, -1, -1, -1, -1, -1, -1, -1};
static const int16_t OF_DEF[29] = {1, 1, 1, 1, 1, 1, 2, 2, 2, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, -1, -1, -1, -1, -1};

typedef struct {
    fse_t ll, of, ml;
    int have_ll, have_of, have_ml;
    huf_t huf;
    int have_huf;
    uint32_t rep[3];
} zstate_t;

/* one sequence table (3.1.1.3.2.2): mode 0 predefined, 1 RLE, 2 FSE, 3 repeat */
static int64_t seq_table(fse_t *f, int *have, int mode, const uint8_t *p, size_t n, int max_sym, int max_al,
                         const int16_t *def, int def_n, int def_al) {
    int16_t norm[256];
    int al, nsym;
    switch (mode) {
    case 0:
        if (fse_build(f, def, def_n, def_al)) return -1;
        *have = 1;
        return 0;
    case 1:
        if (n < 1 || p[0] > max_sym) return -1;
        fse_rle(f, p[0]);
        *have = 1;
        return 1;
    case 2: {
        int64_t u = fse_read_ncount(p, n, max_al, max_sym, norm, &al, &nsym);
        if (u < 0 || fse_build(f, norm, nsym, al)) return -1;
        *have = 1;
        return u;
    }
    default:
        return *have ? 0 : -1;
    }
}

/* 3.1.1.3: one compressed block into out[o..); returns new o or -1 */
static int64_t z_block(zstate_t *z, const uint8_t *p, size_t n, uint8_t *out, size_t o, size_t cap, size_t frame_start) {
    if (n < 1) return -1;
    /* literals section */
    int lt = p[0] & 3, sf = (p[0] >> 2) & 3;
    size_t regen, comp = 0, hdr;
    if (lt <= 1) {
        if (sf == 0 || sf == 2) { regen = p[0] >> 3; hdr = 1; }
        else if (sf == 1) { if (n < 2) return -1; regen = (p[0] >> 4) | ((size_t)p[1] << 4); hdr = 2; }
        else { if (n < 3) return -1; regen = (p[0] >> 4) | ((size_t)p[1] << 4) | ((size_t)p[2] << 12); hdr = 3; }
    } else {
        hdr = sf <= 1 ? 3 : sf == 2 ? 4 : 5;
        if (n < hdr) return -1;
        uint64_t v = 0;
        for (size_t i = 0; i < hdr; i++) v |= (uint64_t)p[i] << (8 * i);
        int bits = sf <= 1 ? 10 : sf == 2 ? 14 : 18;
        regen = (size_t)((v >> 4) & ((1u << bits) - 1));
        comp = (size_t)((v >> (4 + bits)) & ((1u << bits) - 1));
    }
    if (regen > ZBLOCK_MAX) return -1;
    uint8_t *lit = (uint8_t *)malloc(regen + 1);
    if (!lit) return -1;
    size_t q = hdr;
    int64_t rc = -1;
    if (lt == 0) {
        if (n - q < regen) goto done;
        memcpy(lit, p + q, regen);
        q += regen;
    } else if (lt == 1) {
        if (n - q < 1) goto done;
        memset(lit, p[q], regen);
        q += 1;
    } else {
        if (n - q < comp) goto done;
        const uint8_t *cp = p + q;
        size_t cl = comp;
        if (lt == 2) {
            int64_t t = huf_read_tree(&z->huf, cp, cl);
            if (t < 0) goto done;
            z->have_huf = 1;
            cp += t;
            cl -= (size_t)t;
        } else if (!z->have_huf) {
            goto done;
        }
        if (sf == 0) {
            if (huf_stream(&z->huf, cp, cl, lit, regen)) goto done;
        } else {
            if (regen < 6 || cl < 6) goto done;   /* 4 streams need 6 literals (MIN_LITERALS_FOR_4_STREAMS) */
            size_t s1 = cp[0] | ((size_t)cp[1] << 8), s2 = cp[2] | ((size_t)cp[3] << 8), s3 = cp[4] | ((size_t)cp[5] << 8);
            if (6 + s1 + s2 + s3 > cl) goto done;
            size_t s4 = cl - 6 - s1 - s2 - s3, seg = (regen + 3) / 4;
            if (regen < 3 * seg) goto done;
            const uint8_t *b = cp + 6;
            if (huf_stream(&z->huf, b, s1, lit, seg) ||
                huf_stream(&z->huf, b + s1, s2, lit + seg, seg) ||
                huf_stream(&z->huf, b + s1 + s2, s3, lit + 2 * seg, seg) ||
                huf_stream(&z->huf, b + s1 + s2 + s3, s4, lit + 3 * seg, regen - 3 * seg))
                goto done;
        }
        q += comp;
    }
    /* sequences section */
    {
        if (n - q < 1) goto done;
        size_t nseq = p[q];
        if (nseq < 128) q += 1;
        else if (nseq < 255) { if (n - q < 2) goto done; nseq = ((nseq - 128) << 8) + p[q + 1]; q += 2; }
        else { if (n - q < 3) goto done; nseq = p[q + 1] + ((size_t)p[q + 2] << 8) + 0x7F00; q += 3; }
        size_t lpos = 0;
        if (nseq > 0) {
            if (n - q < 1) goto done;
            uint8_t modes = p[q++];
            if (modes & 3) goto done;
            int64_t u;
            u = seq_table(&z->ll, &z->have_ll, modes >> 6, p + q, n - q, 35, 9, LL_DEF, 36, 6);
            if (u < 0) goto done;
            q += (size_t)u;
            u = seq_table(&z->of, &z->have_of, (modes >> 4) & 3, p + q, n - q, 31, 8, OF_DEF, 29, 5);
            if (u < 0) goto done;
            q += (size_t)u;
            u = seq_table(&z->ml, &z->have_ml, (modes >> 2) & 3, p + q, n - q, 52, 9, ML_DEF, 53, 6);
            if (u < 0) goto done;
            q += (size_t)u;
            bwd_t r;
            if (bwd_init(&r, p + q, n - q)) goto done;
            uint32_t sl = bwd_read(&r, z->ll.al), so = bwd_read(&r, z->of.al), sm = bwd_read(&r, z->ml.al);
            for (size_t i = 0; i < nseq; i++) {
                uint32_t ofc = z->of.t[so].sym, mlc = z->ml.t[sm].sym, llc = z->ll.t[sl].sym;
                if (ofc > 31 || mlc > 52 || llc > 35) goto done;
                uint32_t ofv = (1u << ofc) + bwd_read(&r, (int)ofc);
                uint32_t ml = ML_BASE[mlc] + bwd_read(&r, ML_BITS[mlc]);
                uint32_t ll = LL_BASE[llc] + bwd_read(&r, LL_BITS[llc]);
                uint32_t off;
                if (ofv > 3) {
                    off = ofv - 3;
                    z->rep[2] = z->rep[1]; z->rep[1] = z->rep[0]; z->rep[0] = off;
                } else {
                    uint32_t idx = ofv + (ll == 0 ? 1u : 0u);
                    if (idx == 1) off = z->rep[0];
                    else if (idx == 2) { off = z->rep[1]; z->rep[1] = z->rep[0]; z->rep[0] = off; }
                    else if (idx == 3) { off = z->rep[2]; z->rep[2] = z->rep[1]; z->rep[1] = z->rep[0]; z->rep[0] = off; }
                    else {
                        off = z->rep[0] - 1;
                        if (off == 0) goto done;
                        z->rep[2] = z->rep[1]; z->rep[1] = z->rep[0]; z->rep[0] = off;
                    }
                }
                if (i + 1 < nseq) {
                    sl = z->ll.t[sl].base + bwd_read(&r, z->ll.t[sl].nb);
                    sm = z->ml.t[sm].base + bwd_read(&r, z->ml.t[sm].nb);
                    so = z->of.t[so].base + bwd_read(&r, z->of.t[so].nb);
                }
                /* execute (3.1.1.4) */
                if (ll > regen - lpos || ll > cap - o) goto done;
                memcpy(out + o, lit + lpos, ll);
                o += ll;
                lpos += ll;
                if (off > o - frame_start || ml > cap - o) goto done;
                for (uint32_t k = 0; k < ml; k++) out[o + k] = out[o + k - off];
                o += ml;
            }
            if (r.used != r.avail) goto done;
        } else if (q != n) {
            goto done;   /* no sequences: the section is the one byte */
        }
        if (regen - lpos > cap - o) goto done;
        memcpy(out + o, lit + lpos, regen - lpos);
        o += regen - lpos;
        rc = (int64_t)o;
    }
done:
    free(lit);
    return rc;
}

/* One or more frames (decode_all).  Returns the decoded length, -1 on a
 * malformed payload or output beyond cap (zstd_read_bounded). */
int64_t por_zstd_decompress(uint8_t *out, size_t cap, const uint8_t *src, size_t n) {
    size_t i = 0, o = 0;
    if (n == 0) return 0;   /* codec_tagged.rs:209-211 */
    zstate_t *z = (zstate_t *)malloc(sizeof(zstate_t));
    if (!z) return POR_ESMALL;
    int64_t rc = POR_EINVAL;
    while (i < n) {
        if (n - i < 4) goto fail;
        uint32_t magic = zld32(src + i);
        if ((magic & 0xFFFFFFF0u) == 0x184D2A50u) {        /* skippable frame */
            if (n - i < 8) goto fail;
            size_t sz = zld32(src + i + 4);
            if (n - i - 8 < sz) goto fail;
            i += 8 + sz;
            continue;
        }
        if (magic != 0xFD2FB528u) goto fail;
        i += 4;
        if (i >= n) goto fail;
        uint8_t fhd = src[i++];
        int fcs_flag = fhd >> 6, single = (fhd >> 5) & 1, cks = (fhd >> 2) & 1, did = fhd & 3;
        if (fhd & 0x08) goto fail;                          /* reserved bit */
        uint64_t window = 0;
        if (!single) {
            if (i >= n) goto fail;
            uint8_t wd = src[i++];
            int e = wd >> 3, m = wd & 7;
            uint64_t base = 1ull << (10 + e);
            window = base + (base / 8) * (uint64_t)m;
        }
        static const int DID_B[4] = {0, 1, 2, 4};
        if (n - i < (size_t)DID_B[did]) goto fail;
        uint32_t dict = 0;
        for (int k = 0; k < DID_B[did]; k++) dict |= (uint32_t)src[i + k] << (8 * k);
        i += (size_t)DID_B[did];
        if (dict != 0) goto fail;
        int fcs_b = fcs_flag == 0 ? (single ? 1 : 0) : fcs_flag == 1 ? 2 : fcs_flag == 2 ? 4 : 8;
        if (n - i < (size_t)fcs_b) goto fail;
        uint64_t fcs = 0;
        for (int k = 0; k < fcs_b; k++) fcs |= (uint64_t)src[i + k] << (8 * k);
        if (fcs_b == 2) fcs += 256;
        i += (size_t)fcs_b;
        if (single) window = fcs;
        if (window > (1ull << 27) + 1) goto fail;
        uint64_t bmax = window < ZBLOCK_MAX ? window : ZBLOCK_MAX;
        memset(z, 0, sizeof(*z));
        z->rep[0] = 1; z->rep[1] = 4; z->rep[2] = 8;
        size_t start = o;
        for (;;) {
            if (n - i < 3) goto fail;
            uint32_t bh = src[i] | ((uint32_t)src[i + 1] << 8) | ((uint32_t)src[i + 2] << 16);
            i += 3;
            int last = bh & 1, bt = (bh >> 1) & 3;
            size_t bs = bh >> 3;
            if (bt == 3) goto fail;
            if (bt == 1) {
                if (bs > bmax || n - i < 1 || bs > cap - o) goto fail;
                memset(out + o, src[i], bs);
                o += bs;
                i += 1;
            } else {
                if (bs > bmax || n - i < bs) goto fail;
                if (bt == 0) {
                    if (bs > cap - o) goto fail;
                    memcpy(out + o, src + i, bs);
                    o += bs;
                } else {
                    size_t lim = cap - o < bmax ? cap - o : (size_t)bmax;
                    int64_t r = z_block(z, src + i, bs, out, o, o + lim, start);
                    if (r < 0) goto fail;
                    o = (size_t)r;
                }
                i += bs;
            }
            if (last) break;
        }
        if (fcs_b && (uint64_t)(o - start) != fcs) goto fail;
        if (cks) {
            if (n - i < 4) goto fail;
            uint32_t want = zld32(src + i);
            if ((uint32_t)por_xxh64(out + start, o - start, 0) != want) goto fail;
            i += 4;
        }
    }
    rc = (int64_t)o;
fail:
    free(z);
    return rc;
}
