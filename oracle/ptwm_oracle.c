/*
 * ptwm_oracle.c -- CPU restatement of the PTWM plane-codec hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker and the timed CPU baseline); see
 * ptwm_oracle.h.  Citations are file:line under crates/ptwm-core/src/ of the
 * reference tree.  Arithmetic follows the reference's integer widths,
 * including its wrapping u8 bit counter in the Huffman reader (release
 * builds of the reference do not check overflow: Cargo.toml [profile.release]
 * leaves overflow-checks off).
 *
 * Parity pinning (what checks each part) is listed in tests/test_oracle_*.py.
 */
#define _POSIX_C_SOURCE 200809L   /* pthread barriers under -std=c11 */
#include "ptwm_oracle.h"

#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* bit reorder: split/dtype8.rs:30-62, dtype16.rs:11-59, dtype32.rs:13-55     */
/* ------------------------------------------------------------------------- */

uint8_t por_reorder_e4m3(uint8_t v) { return (uint8_t)(((v & 0x78) << 1) | ((v & 0x80) >> 4) | (v & 0x07)); }
uint8_t por_revert_e4m3(uint8_t v) { return (uint8_t)(((v & 0xF0) >> 1) | ((v & 0x08) << 4) | (v & 0x07)); }
uint8_t por_reorder_e5m2(uint8_t v) { return (uint8_t)(((v & 0x7C) << 1) | ((v & 0x80) >> 5) | (v & 0x03)); }
uint8_t por_revert_e5m2(uint8_t v) { return (uint8_t)(((v & 0xF8) >> 1) | ((v & 0x04) << 5) | (v & 0x03)); }

uint32_t por_reorder16x2(uint32_t v) {
    return ((v << 1) & 0xFF00FF00u) | ((v >> 8) & 0x00800080u) | (v & 0x007F007Fu);
}
uint32_t por_revert16x2(uint32_t v) {
    return ((v << 8) & 0x80008000u) | ((v >> 1) & 0x7F807F80u) | (v & 0x007F007Fu);
}
uint32_t por_reorder32(uint32_t v) {
    return ((v << 1) & 0xFF000000u) | ((v >> 8) & 0x00800000u) | (v & 0x007FFFFFu);
}
uint32_t por_revert32(uint32_t v) {
    return ((v << 8) & 0x80000000u) | ((v >> 1) & 0x7F800000u) | (v & 0x007FFFFFu);
}

static uint32_t ld32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
static void st32(uint8_t *p, uint32_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); p[2] = (uint8_t)(v >> 16); p[3] = (uint8_t)(v >> 24); }
static uint64_t ld64(const uint8_t *p) { return (uint64_t)ld32(p) | ((uint64_t)ld32(p + 4) << 32); }

/* dtype16.rs:31-59 -- only floor(len/4) words; a trailing element is left as is */
void por_reorder16_buf(uint8_t *d, size_t len) { for (size_t i = 0; i + 4 <= len; i += 4) st32(d + i, por_reorder16x2(ld32(d + i))); }
void por_revert16_buf(uint8_t *d, size_t len) { for (size_t i = 0; i + 4 <= len; i += 4) st32(d + i, por_revert16x2(ld32(d + i))); }
/* dtype32.rs:28-55 */
void por_reorder32_buf(uint8_t *d, size_t len) { for (size_t i = 0; i + 4 <= len; i += 4) st32(d + i, por_reorder32(ld32(d + i))); }
void por_revert32_buf(uint8_t *d, size_t len) { for (size_t i = 0; i + 4 <= len; i += 4) st32(d + i, por_revert32(ld32(d + i))); }

/* ------------------------------------------------------------------------- */
/* byte / nibble split: transforms/byte_split.rs:86-176, nibble_split.rs:72-120 */
/* ------------------------------------------------------------------------- */

void por_byte_split(const uint8_t *in, size_t len, int n, uint8_t *const *planes) {
    for (size_t j = 0; j < len; j++) planes[j % (size_t)n][j / (size_t)n] = in[j];
}
void por_byte_merge(const uint8_t *const *planes, size_t plane_len, int n, uint8_t *out) {
    for (int p = 0; p < n; p++)
        for (size_t j = 0; j < plane_len; j++) out[j * (size_t)n + (size_t)p] = planes[p][j];
}
void por_nibble_split(const uint8_t *in, size_t len, uint8_t *hi, uint8_t *lo) {
    for (size_t i = 0; i < len; i++) { hi[i] = (in[i] >> 4) & 0x0F; lo[i] = in[i] & 0x0F; }
}
void por_nibble_merge(const uint8_t *hi, const uint8_t *lo, size_t len, uint8_t *out) {
    for (size_t i = 0; i < len; i++) out[i] = (uint8_t)(((hi[i] & 0x0F) << 4) | (lo[i] & 0x0F));
}

/* ------------------------------------------------------------------------- */
/* fused chains: transforms/fusion.rs:32-519                                  */
/* ------------------------------------------------------------------------- */

int por_chain_nplanes(int chain) {
    switch (chain) {
    case POR_CHAIN_IEEE16_SPLIT2: return 2;
    case POR_CHAIN_IEEE32_SPLIT4: return 4;
    case POR_CHAIN_E4M3_NIBBLE: case POR_CHAIN_E5M2_NIBBLE: case POR_CHAIN_NIBBLE_SPLIT: return 2;
    case POR_CHAIN_PASSTHROUGH: return 1;
    default: return -1;
    }
}

int64_t por_chain_plane_len(int chain, size_t len) {
    switch (chain) {
    case POR_CHAIN_IEEE16_SPLIT2: return (len % 2) ? -1 : (int64_t)(len / 2);   /* fusion.rs:37-42 */
    case POR_CHAIN_IEEE32_SPLIT4: return (len % 4) ? -1 : (int64_t)(len / 4);   /* fusion.rs:209-215 */
    case POR_CHAIN_E4M3_NIBBLE: case POR_CHAIN_E5M2_NIBBLE: case POR_CHAIN_NIBBLE_SPLIT:
    case POR_CHAIN_PASSTHROUGH: return (int64_t)len;
    default: return -1;
    }
}

int por_chain_forward(int chain, const uint8_t *src, size_t len, uint8_t *const *pl) {
    size_t i;
    switch (chain) {
    case POR_CHAIN_IEEE16_SPLIT2: { /* fusion.rs:35-94 */
        if (len % 2) return POR_EINVAL;
        size_t words = len / 4;
        for (i = 0; i < words; i++) {
            uint32_t r = por_reorder16x2(ld32(src + 4 * i));
            pl[0][2 * i] = (uint8_t)r; pl[1][2 * i] = (uint8_t)(r >> 8);
            pl[0][2 * i + 1] = (uint8_t)(r >> 16); pl[1][2 * i + 1] = (uint8_t)(r >> 24);
        }
        if (len % 4 == 2) { /* trailing element IS reordered here (fusion.rs:73-89) */
            size_t k = len - 2;
            uint16_t v = (uint16_t)(src[k] | (src[k + 1] << 8));
            uint16_t r = (uint16_t)(((v << 1) & 0xFF00) | ((v >> 8) & 0x0080) | (v & 0x007F));
            pl[0][len / 2 - 1] = (uint8_t)r; pl[1][len / 2 - 1] = (uint8_t)(r >> 8);
        }
        return 0;
    }
    case POR_CHAIN_IEEE32_SPLIT4: /* fusion.rs:208-255 */
        if (len % 4) return POR_EINVAL;
        for (i = 0; i < len / 4; i++) {
            uint32_t r = por_reorder32(ld32(src + 4 * i));
            pl[0][i] = (uint8_t)r; pl[1][i] = (uint8_t)(r >> 8); pl[2][i] = (uint8_t)(r >> 16); pl[3][i] = (uint8_t)(r >> 24);
        }
        return 0;
    case POR_CHAIN_E4M3_NIBBLE: /* fusion.rs:329-338 */
        for (i = 0; i < len; i++) { uint8_t r = por_reorder_e4m3(src[i]); pl[0][i] = r >> 4; pl[1][i] = r & 0x0F; }
        return 0;
    case POR_CHAIN_E5M2_NIBBLE: /* fusion.rs:431-440 */
        for (i = 0; i < len; i++) { uint8_t r = por_reorder_e5m2(src[i]); pl[0][i] = r >> 4; pl[1][i] = r & 0x0F; }
        return 0;
    case POR_CHAIN_NIBBLE_SPLIT: por_nibble_split(src, len, pl[0], pl[1]); return 0;
    case POR_CHAIN_PASSTHROUGH: if (len) memcpy(pl[0], src, len); return 0;
    default: return POR_EUNSUP;
    }
}

int por_chain_inverse(int chain, const uint8_t *const *pl, size_t n, uint8_t *out) {
    size_t i;
    switch (chain) {
    case POR_CHAIN_IEEE16_SPLIT2: { /* fusion.rs:127-194 */
        for (i = 0; i < n / 2; i++) {
            uint32_t r = (uint32_t)pl[0][2 * i] | ((uint32_t)pl[1][2 * i] << 8) |
                         ((uint32_t)pl[0][2 * i + 1] << 16) | ((uint32_t)pl[1][2 * i + 1] << 24);
            st32(out + 4 * i, por_revert16x2(r));
        }
        if (n % 2) {
            size_t k = n - 1;
            uint16_t r = (uint16_t)(pl[0][k] | (pl[1][k] << 8));
            uint16_t v = (uint16_t)(((r << 8) & 0x8000) | ((r >> 1) & 0x7F80) | (r & 0x007F));
            out[2 * k] = (uint8_t)v; out[2 * k + 1] = (uint8_t)(v >> 8);
        }
        return 0;
    }
    case POR_CHAIN_IEEE32_SPLIT4: /* fusion.rs:261-315 */
        for (i = 0; i < n; i++) {
            uint32_t r = (uint32_t)pl[0][i] | ((uint32_t)pl[1][i] << 8) | ((uint32_t)pl[2][i] << 16) | ((uint32_t)pl[3][i] << 24);
            st32(out + 4 * i, por_revert32(r));
        }
        return 0;
    case POR_CHAIN_E4M3_NIBBLE: /* fusion.rs:376-399 */
        for (i = 0; i < n; i++) out[i] = por_revert_e4m3((uint8_t)(((pl[0][i] & 0x0F) << 4) | (pl[1][i] & 0x0F)));
        return 0;
    case POR_CHAIN_E5M2_NIBBLE: /* fusion.rs:478-501 */
        for (i = 0; i < n; i++) out[i] = por_revert_e5m2((uint8_t)(((pl[0][i] & 0x0F) << 4) | (pl[1][i] & 0x0F)));
        return 0;
    case POR_CHAIN_NIBBLE_SPLIT: por_nibble_merge(pl[0], pl[1], n, out); return 0;
    case POR_CHAIN_PASSTHROUGH: if (n) memcpy(out, pl[0], n); return 0;
    default: return POR_EUNSUP;
    }
}

/* ------------------------------------------------------------------------- */
/* plane ops on one terminal plane (chain/dispatch.rs:96-122)                 */
/* ------------------------------------------------------------------------- */

/* little-endian element i of width w (1, 2, 4, 8) */
static uint64_t ld_elem(const uint8_t *p, unsigned w) {
    uint64_t v = 0;
    for (unsigned k = 0; k < w; ++k) v |= (uint64_t)p[k] << (8 * k);
    return v;
}
static void st_elem(uint8_t *p, unsigned w, uint64_t v) {
    for (unsigned k = 0; k < w; ++k) p[k] = (uint8_t)(v >> (8 * k));
}
static uint64_t width_mask(unsigned w) { return w == 8 ? ~0ull : (1ull << (8 * w)) - 1; }
static int width_ok(unsigned w, size_t len) { return (w == 1 || w == 2 || w == 4 || w == 8) && len % w == 0; }

/* IntDelta (transforms/int_delta.rs:38-46, 134-226): out[0] = in[0],
 * out[i] = in[i] - in[i-1] (wrapping at the element width); the inverse is
 * the running wrapping sum.  A length that is not a multiple of the width
 * is InvalidContainer (:77-83, :104-110). */
int por_int_delta(const uint8_t *in, size_t len, unsigned width, int inverse, uint8_t *out) {
    if (!width_ok(width, len)) return POR_EINVAL;
    const uint64_t m = width_mask(width);
    uint64_t prev = 0;
    for (size_t i = 0; i < len; i += width) {
        const uint64_t v = ld_elem(in + i, width);
        if (inverse) {
            prev = i == 0 ? v : (prev + v) & m;
            st_elem(out + i, width, prev);
        } else {
            st_elem(out + i, width, i == 0 ? v : (v - prev) & m);
            prev = v;
        }
    }
    return 0;
}

/* PredictorXor (transforms/predictor_xor.rs:10-25, 192-246): a 2^16-entry
 * table of past values, zeroed per plane; per element the prediction is
 * table[hash], the residual value ^ prediction, then table[hash] = value
 * and hash = ((hash << 6) ^ value) & 0xFFFF, starting from hash 0.  The
 * inverse runs the same recurrence on the recovered values. */
int por_predictor_xor(const uint8_t *in, size_t len, unsigned width, int inverse, uint8_t *out) {
    if (!width_ok(width, len)) return POR_EINVAL;
    if (len == 0) return 0;
    uint64_t *table = (uint64_t *)calloc(1u << 16, sizeof(uint64_t));
    if (!table) return POR_ESMALL;
    uint64_t hash = 0;
    for (size_t i = 0; i < len; i += width) {
        const uint64_t x = ld_elem(in + i, width);
        const uint64_t pred = table[hash];
        const uint64_t value = inverse ? x ^ pred : x;
        st_elem(out + i, width, x ^ pred);
        table[hash] = value;
        hash = ((hash << 6) ^ value) & 0xFFFFu;
    }
    free(table);
    return 0;
}

/* MantissaZeroStrip (transforms/mantissa_zero.rs): k in 1..=7 (new(),
 * chain/dispatch.rs:96-104); forward b >> k, refused when any byte has a
 * nonzero low k bits; inverse b << k (u8, high bits dropped). */
int por_mantissa_zero_strip(const uint8_t *in, size_t len, unsigned k, int inverse, uint8_t *out) {
    if (k < 1 || k > 7) return POR_EINVAL;
    const uint8_t low = (uint8_t)((1u << k) - 1);
    if (!inverse)
        for (size_t i = 0; i < len; ++i)
            if (in[i] & low) return POR_EINVAL;
    for (size_t i = 0; i < len; ++i) out[i] = inverse ? (uint8_t)(in[i] << k) : (uint8_t)(in[i] >> k);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* entropy helpers: entropy/mod.rs:34-40, stream_frame.rs:27-62               */
/* ------------------------------------------------------------------------- */

void por_histogram(const uint8_t *d, size_t len, uint32_t h[256]) {
    memset(h, 0, 256 * sizeof(uint32_t));
    for (size_t i = 0; i < len; i++) h[d[i]]++;
}

void por_split_four(size_t len, size_t s[4], size_t e[4]) {
    size_t base = len / 4, rem = len % 4, start = 0;
    for (int i = 0; i < 4; i++) { size_t l = base + ((size_t)i < rem); s[i] = start; e[i] = start + l; start += l; }
}

/* ------------------------------------------------------------------------- */
/* Huffman tree: entropy/huffman/tree.rs                                      */
/* ------------------------------------------------------------------------- */

#define HUF_MAX_TABLE_LOG 11

/* min-heap over (freq, id); keys are distinct, so the pop order matches any
 * correct priority queue, including Rust's BinaryHeap<Reverse<(u64,usize)>> */
typedef struct { uint64_t f; uint32_t id; } hkey;
static int hless(hkey a, hkey b) { return a.f < b.f || (a.f == b.f && a.id < b.id); }
static void hpush(hkey *h, int *n, hkey k) {
    int i = (*n)++;
    h[i] = k;
    while (i > 0) { int p = (i - 1) / 2; if (!hless(h[i], h[p])) break; hkey t = h[i]; h[i] = h[p]; h[p] = t; i = p; }
}
static hkey hpop(hkey *h, int *n) {
    hkey top = h[0];
    h[0] = h[--(*n)];
    int i = 0;
    for (;;) {
        int l = 2 * i + 1, r = l + 1, m = i;
        if (l < *n && hless(h[l], h[m])) m = l;
        if (r < *n && hless(h[r], h[m])) m = r;
        if (m == i) break;
        hkey t = h[i]; h[i] = h[m]; h[m] = t; i = m;
    }
    return top;
}

/* tree.rs:212-242 */
static void enforce_max_code_length(uint8_t *lengths, uint8_t max_len) {
    int clamped = 0;
    for (int s = 0; s < 256; s++) if (lengths[s] > max_len) { lengths[s] = max_len; clamped = 1; }
    if (!clamped) return;
    uint32_t cap = 1u << max_len;
    for (;;) {
        uint32_t kraft = 0;
        for (int s = 0; s < 256; s++) if (lengths[s]) kraft += 1u << (max_len - lengths[s]);
        if (kraft <= cap) break;
        int victim = -1;
        for (int s = 0; s < 256; s++)  /* min_by_key keeps the first minimum */
            if (lengths[s] > 0 && lengths[s] < max_len && (victim < 0 || lengths[s] < lengths[victim])) victim = s;
        if (victim < 0) break;
        lengths[victim]++;
    }
}

/* tree.rs:19-85 with enforce_max_code_length (tree.rs:212-242) at max_len */
int por_huf_lengths_limited(const uint32_t freqs[256], uint8_t lengths[256], int max_len) {
    int sym[256], n = 0;
    memset(lengths, 0, 256);
    for (int i = 0; i < 256; i++) if (freqs[i] > 0) sym[n++] = i;
    if (n == 0) return 0;
    if (n == 1) { lengths[sym[0]] = 1; return 1; }
    uint64_t nf[512];
    int left[512], right[512];
    hkey heap[512];
    int hn = 0;
    for (int id = 0; id < n; id++) { nf[id] = freqs[sym[id]]; hpush(heap, &hn, (hkey){nf[id], (uint32_t)id}); }
    int next = n;
    while (hn > 1) {
        hkey a = hpop(heap, &hn), b = hpop(heap, &hn);
        nf[next] = a.f + b.f; left[next] = (int)a.id; right[next] = (int)b.id;
        hpush(heap, &hn, (hkey){a.f + b.f, (uint32_t)next});
        next++;
    }
    int root = (int)hpop(heap, &hn).id;
    int stack_id[512]; uint8_t stack_d[512]; int sp = 0;
    stack_id[sp] = root; stack_d[sp] = 0; sp++;
    while (sp > 0) {
        sp--; int id = stack_id[sp]; uint8_t d = stack_d[sp];
        if (id < n) lengths[sym[id]] = d;
        else {
            uint8_t nd = d == 255 ? 255 : (uint8_t)(d + 1);
            stack_id[sp] = left[id]; stack_d[sp] = nd; sp++;
            stack_id[sp] = right[id]; stack_d[sp] = nd; sp++;
        }
    }
    enforce_max_code_length(lengths, (uint8_t)max_len);
    return 1;
}

/* tree.rs:19-85 + :212-242, the reference encoder's 11-bit limit */
int por_huf_lengths_from_freqs(const uint32_t freqs[256], uint8_t lengths[256]) {
    return por_huf_lengths_limited(freqs, lengths, HUF_MAX_TABLE_LOG);
}

static uint16_t reverse_bits(uint16_t code, int nbits) {
    uint16_t out = 0;
    for (int i = 0; i < nbits; i++) { out = (uint16_t)((out << 1) | (code & 1)); code >>= 1; }
    return out;
}

/* tree.rs:102-177: returns max_bits, or 0 for None */
int por_huf_from_lengths(const uint8_t lengths[256], uint16_t *table, uint16_t rev_codes[256]) {
    int max_bits = 0;
    for (int s = 0; s < 256; s++) if (lengths[s] > max_bits) max_bits = lengths[s];
    if (max_bits < 1) max_bits = 1;
    if (max_bits > HUF_MAX_TABLE_LOG) return 0;
    uint16_t counts[HUF_MAX_TABLE_LOG + 1] = {0};
    uint32_t total = 0;
    for (int s = 0; s < 256; s++) if (lengths[s]) { counts[lengths[s]]++; total++; }
    if (total == 0) return 0;
    uint16_t next_code[HUF_MAX_TABLE_LOG + 1] = {0};
    uint16_t code = 0;
    for (int b = 1; b <= max_bits; b++) {
        code = (uint16_t)((code + counts[b - 1]) << 1);
        if (code > (1u << b)) return 0;
        next_code[b] = code;
    }
    uint16_t codes[256] = {0};
    for (int s = 0; s < 256; s++) {
        int l = lengths[s];
        if (!l) continue;
        uint16_t c = next_code[l];
        if (c >= (1u << l)) return 0;
        codes[s] = c; next_code[l] = (uint16_t)(c + 1);
    }
    size_t tsize = (size_t)1 << max_bits;
    uint16_t fallback = (uint16_t)(max_bits << 8);
    for (size_t i = 0; i < tsize; i++) table[i] = fallback;
    for (int s = 0; s < 256; s++) {
        int l = lengths[s];
        if (!l) continue;
        uint16_t rev = reverse_bits(codes[s], l);
        if (rev_codes) rev_codes[s] = rev;
        uint16_t entry = (uint16_t)((l << 8) | s);
        for (size_t i = 0; i < ((size_t)1 << (max_bits - l)); i++) {
            size_t idx = rev | (i << l);
            if (table[idx] != fallback && table[idx] != entry) return 0;
            table[idx] = entry;
        }
    }
    return max_bits;
}

/* weights.rs:8-32 */
int64_t por_huf_encode_weights(const uint8_t *w, size_t n, uint8_t *out, size_t cap) {
    if (n == 0 || n > 256) return POR_EINVAL;
    size_t need = (n <= 127 ? 1 : 2) + (n + 1) / 2, o = 0;
    if (need > cap) return POR_ESMALL;
    if (n <= 127) out[o++] = (uint8_t)(0x80 | n);
    else { out[o++] = 0x80; out[o++] = (uint8_t)n; }
    for (size_t i = 0; i < n; i += 2) {
        uint8_t lo = w[i] & 0x0F, hi = (i + 1 < n) ? (w[i + 1] & 0x0F) : 0;
        out[o++] = (uint8_t)(lo | (hi << 4));
    }
    return (int64_t)o;
}

/* weights.rs:34-85 */
int64_t por_huf_decode_weights(const uint8_t *src, size_t len, uint8_t w[256], int *n_out) {
    if (len == 0) return POR_EINVAL;
    uint8_t h = src[0];
    if (!(h & 0x80)) return POR_EINVAL;
    size_t n, hb;
    if (h == 0x80) {
        if (len < 2) return POR_EINVAL;
        n = src[1] ? src[1] : 256;
        if (n < 128) return POR_EINVAL;
        hb = 2;
    } else {
        n = h & 0x7F;
        if (n == 0) return POR_EINVAL;
        hb = 1;
    }
    size_t need = hb + (n + 1) / 2;
    if (len < need) return POR_EINVAL;
    for (size_t i = 0; i < n; i++) { uint8_t b = src[hb + i / 2]; w[i] = (i % 2 == 0) ? (b & 0x0F) : ((b >> 4) & 0x0F); }
    *n_out = (int)n;
    return (int64_t)need;
}

/* ------------------------------------------------------------------------- */
/* backward bitstream: entropy/huffman/bitstream.rs                           */
/* ------------------------------------------------------------------------- */

typedef struct { uint8_t *buf; size_t ptr; uint64_t cont; uint32_t cnt; } bw_t;

/* bitstream.rs:22-35 */
static void bw_write(bw_t *w, uint16_t bits, uint8_t nbits) {
    w->cont |= (uint64_t)bits << w->cnt;
    w->cnt += nbits;
    if (w->cnt >= 32) {
        w->ptr -= 4;
        uint32_t v = (uint32_t)w->cont; /* BE: lowest bits land at the highest index */
        w->buf[w->ptr] = (uint8_t)(v >> 24); w->buf[w->ptr + 1] = (uint8_t)(v >> 16);
        w->buf[w->ptr + 2] = (uint8_t)(v >> 8); w->buf[w->ptr + 3] = (uint8_t)v;
        w->cont >>= 32; w->cnt -= 32;
    }
}
/* bitstream.rs:40-50 */
static size_t bw_finish(bw_t *w) {
    while (w->cnt > 0) {
        w->ptr -= 1;
        w->buf[w->ptr] = (uint8_t)(w->cont & 0xFF);
        w->cont >>= 8;
        w->cnt = w->cnt >= 8 ? w->cnt - 8 : 0;
    }
    return w->ptr;
}

int64_t por_bitwriter_pack(const uint16_t *bits, const uint8_t *nbits, size_t n, uint8_t *out, size_t cap) {
    size_t total = 0;
    for (size_t i = 0; i < n; i++) total += nbits[i];
    size_t scratch_len = (total + 7) / 8 + 8;
    uint8_t *scratch = (uint8_t *)calloc(scratch_len, 1);
    if (!scratch) return POR_ESMALL;
    bw_t w = {scratch, scratch_len, 0, 0};
    for (size_t i = 0; i < n; i++) bw_write(&w, bits[i], nbits[i]);
    size_t start = bw_finish(&w), m = scratch_len - start;
    if (m > cap) { free(scratch); return POR_ESMALL; }
    memcpy(out, scratch + start, m);
    free(scratch);
    return (int64_t)m;
}

typedef struct { const uint8_t *data; int64_t bi; uint64_t cont; uint8_t cnt; } br_t;

/* bitstream.rs:63-82 */
static void br_init(br_t *r, const uint8_t *d, size_t n) {
    r->data = d; r->bi = (int64_t)n - 1; r->cont = 0; r->cnt = 0;
    int64_t avail = r->bi + 1; if (avail > 8) avail = 8;
    for (int64_t i = 0; i < avail; i++) { r->cont |= (uint64_t)d[r->bi] << r->cnt; r->cnt = (uint8_t)(r->cnt + 8); r->bi--; }
}
/* bitstream.rs:88-106 */
static void br_reload(br_t *r) {
    if (r->cnt == 0 && r->bi >= 7) {
        const uint8_t *p = r->data + r->bi - 7;
        uint64_t w = 0;
        for (int i = 0; i < 8; i++) w = (w << 8) | p[i];
        r->cont = w; r->cnt = 64; r->bi -= 8;
    } else if (r->cnt <= 32 && r->bi >= 3) {
        const uint8_t *p = r->data + r->bi - 3;
        uint32_t w = ((uint32_t)p[0] << 24) | ((uint32_t)p[1] << 16) | ((uint32_t)p[2] << 8) | p[3];
        r->cont |= (uint64_t)w << r->cnt; r->cnt = (uint8_t)(r->cnt + 32); r->bi -= 4;
    }
}
/* bitstream.rs:108-121 */
static void br_refill(br_t *r) {
    if (r->cnt <= 32 && r->bi >= 3) br_reload(r);
    else while (r->cnt < 56 && r->bi >= 0) { r->cont |= (uint64_t)r->data[r->bi] << r->cnt; r->cnt = (uint8_t)(r->cnt + 8); r->bi--; }
}
/* bitstream.rs:129-137 -- the u8 counter wraps on malformed input */
static uint8_t br_decode(br_t *r, const uint16_t *table, uint64_t mask) {
    uint16_t e = table[r->cont & mask];
    uint8_t nb = (uint8_t)(e >> 8);
    r->cont >>= nb; r->cnt = (uint8_t)(r->cnt - nb);
    return (uint8_t)(e & 0xFF);
}
static void br_refill_to(br_t *r, uint8_t nbits) {
    while (r->cnt < nbits && r->bi >= 0) { r->cont |= (uint64_t)r->data[r->bi] << r->cnt; r->cnt = (uint8_t)(r->cnt + 8); r->bi--; }
}
static size_t br_avail(const br_t *r) { return (size_t)r->cnt + (size_t)(r->bi + 1 > 0 ? r->bi + 1 : 0) * 8; }
static int br_exhausted(const br_t *r) { return r->bi < 0 && r->cont == 0; }

/* ------------------------------------------------------------------------- */
/* Huffman compress: entropy/huffman/compress.rs:9-103                        */
/* ------------------------------------------------------------------------- */

int64_t por_huf_compress(uint8_t *dst, size_t cap, const uint8_t *src, size_t len, int *outcome) {
    *outcome = POR_OUT_INCOMPRESSIBLE;
    if (len == 0) return 0;
    uint32_t freqs[256];
    por_histogram(src, len, freqs);
    uint8_t lengths[256];
    uint16_t table[1 << HUF_MAX_TABLE_LOG], rev[256];
    if (!por_huf_lengths_from_freqs(freqs, lengths)) return 0;
    int max_bits = por_huf_from_lengths(lengths, table, rev);
    if (!max_bits) return 0;
    int n = 0;
    for (int s = 0; s < 256; s++) if (lengths[s]) n = s + 1;
    uint8_t hdr[2 + 128 + 16];
    int64_t wl = por_huf_encode_weights(lengths, (size_t)n, hdr, sizeof(hdr));
    if (wl < 0) return 0;
    size_t jt = (size_t)wl, header_len = jt + 16;
    memset(hdr + jt, 0, 16);
    if (header_len >= cap) { *outcome = POR_OUT_DST_TOO_SMALL; return 0; }
    memcpy(dst, hdr, header_len);
    size_t s[4], e[4];
    por_split_four(len, s, e);
    size_t max_seg = 0;
    for (int i = 0; i < 4; i++) if (e[i] - s[i] > max_seg) max_seg = e[i] - s[i];
    size_t max_out = (max_seg * (size_t)max_bits + 7) / 8 + 8;
    uint8_t *scratch = (uint8_t *)malloc(max_out);
    if (!scratch) return POR_ESMALL;
    uint32_t lens[4];
    size_t off = header_len;
    for (int i = 0; i < 4; i++) {
        bw_t w = {scratch, max_out, 0, 0};
        for (size_t k = s[i]; k < e[i]; k++) bw_write(&w, rev[src[k]], lengths[src[k]]);
        size_t start = bw_finish(&w), written = max_out - start;
        if (off + written > cap) { free(scratch); *outcome = POR_OUT_DST_TOO_SMALL; return 0; }
        if (written > 0xFFFFFFFFu) { free(scratch); *outcome = POR_OUT_LEN_OVERFLOW; return 0; }
        memcpy(dst + off, scratch + start, written);
        off += written;
        lens[i] = (uint32_t)written;
    }
    free(scratch);
    if (off >= len) { *outcome = POR_OUT_NOT_BENEFICIAL; return 0; }
    for (int i = 0; i < 4; i++) st32(dst + jt + 4 * i, lens[i]);
    *outcome = POR_OUT_ENCODED;
    return (int64_t)off;
}

/* ------------------------------------------------------------------------- */
/* Huffman decompress: entropy/huffman/decompress.rs:8-211, mod.rs:34-43      */
/* ------------------------------------------------------------------------- */

/* decompress.rs:152-211 */
static int huf_tail(br_t *r, const uint16_t *table, uint64_t mask, uint8_t max_bits, uint8_t *out, size_t len) {
    size_t i = 0;
    while (i < len && r->bi >= 3) {
        if (r->cnt < max_bits) br_refill(r);
        out[i++] = br_decode(r, table, mask);
    }
    size_t tsize = (size_t)1 << max_bits;
    while (i < len) {
        size_t avail = br_avail(r);
        if (avail == 0) return POR_EINVAL;
        br_refill_to(r, max_bits);              /* peek_bits */
        if (r->cnt == 0) return POR_EINVAL;
        size_t idx = (size_t)(r->cont & (((uint64_t)1 << max_bits) - 1));
        if (idx >= tsize) return POR_EINVAL;
        uint16_t e = table[idx];
        uint8_t nb = (uint8_t)(e >> 8), sym = (uint8_t)(e & 0xFF);
        if ((size_t)nb > avail) return POR_EINVAL;
        if (nb) {                               /* consume */
            if (r->cnt < nb) br_refill_to(r, nb);
            if (r->cnt < nb) return POR_EINVAL;
            r->cont >>= nb; r->cnt = (uint8_t)(r->cnt - nb);
        }
        out[i++] = sym;
    }
    return 0;
}

int64_t por_huf_decompress(uint8_t *dst, size_t dst_len, const uint8_t *src, size_t src_len) {
    uint8_t w[256];
    int n = 0;
    int64_t pos = por_huf_decode_weights(src, src_len, w, &n);
    if (pos < 0) return POR_EINVAL;
    uint8_t lengths[256] = {0};
    for (int i = 0; i < n; i++) { if (w[i] > HUF_MAX_TABLE_LOG) return POR_EINVAL; lengths[i] = w[i]; }
    uint16_t table[1 << HUF_MAX_TABLE_LOG];
    int max_bits = por_huf_from_lengths(lengths, table, NULL);
    if (!max_bits) return POR_EINVAL;
    size_t p = (size_t)pos;
    if (src_len - p < 16) return POR_EINVAL;
    uint64_t lens[4], total = 0;
    for (int i = 0; i < 4; i++) { lens[i] = ld32(src + p + 4 * i); total += lens[i]; }
    p += 16;
    if (total != (uint64_t)(src_len - p)) return POR_EINVAL;
    br_t r[4];
    size_t so = p;
    for (int i = 0; i < 4; i++) { br_init(&r[i], src + so, (size_t)lens[i]); so += (size_t)lens[i]; }
    size_t s[4], e[4];
    por_split_four(dst_len, s, e);
    uint64_t mask = ((uint64_t)1 << max_bits) - 1;
    size_t op[4] = {s[0], s[1], s[2], s[3]}, fe[4];
    for (int i = 0; i < 4; i++) fe[i] = e[i] >= 3 ? e[i] - 3 : 0;
    while (op[0] < fe[0] && op[1] < fe[1] && op[2] < fe[2] && op[3] < fe[3] &&
           r[0].bi >= 3 && r[1].bi >= 3 && r[2].bi >= 3 && r[3].bi >= 3) {
        for (int round = 0; round < 2; round++) {
            for (int i = 0; i < 4; i++) br_refill(&r[i]);
            for (int k = 0; k < 2; k++)
                for (int i = 0; i < 4; i++) dst[op[i]++] = br_decode(&r[i], table, mask);
        }
    }
    for (int i = 0; i < 4; i++)
        if (huf_tail(&r[i], table, mask, (uint8_t)max_bits, dst + op[i], e[i] - op[i]) < 0) return POR_EINVAL;
    for (int i = 0; i < 4; i++) if (!br_exhausted(&r[i])) return POR_EINVAL;
    return (int64_t)dst_len;
}

/* ------------------------------------------------------------------------- */
/* rANS: entropy/rans/compress.rs, decompress.rs                              */
/* ------------------------------------------------------------------------- */

#define RANS_PROB_BITS 11
#define RANS_PROB_SCALE (1u << RANS_PROB_BITS)
#define RANS_L (1u << 23)

/* compress.rs:72-122 */
int por_rans_normalize(const uint32_t raw[256], uint16_t f[256], uint16_t cum[256]) {
    uint64_t total = 0;
    for (int i = 0; i < 256; i++) total += raw[i];
    memset(f, 0, 512); memset(cum, 0, 512);
    if (total == 0) return 0;
    uint32_t assigned = 0;
    int max_sym = 0, max_freq_sym = 0;
    for (int i = 0; i < 256; i++) {
        if (raw[i] > 0) {
            uint64_t v = ((uint64_t)raw[i] * RANS_PROB_SCALE) / total;
            if (v < 1) v = 1;
            f[i] = (uint16_t)v;
            assigned += f[i];
            max_sym = i;
            if (raw[i] > raw[max_freq_sym]) max_freq_sym = i;
        }
    }
    if (assigned > RANS_PROB_SCALE) {
        uint32_t excess = assigned - RANS_PROB_SCALE;
        if ((uint32_t)f[max_freq_sym] > excess) f[max_freq_sym] = (uint16_t)(f[max_freq_sym] - excess);
        else return 0;
    } else if (assigned < RANS_PROB_SCALE) {
        f[max_freq_sym] = (uint16_t)(f[max_freq_sym] + (RANS_PROB_SCALE - assigned));
    }
    uint16_t run = 0;
    for (int i = 0; i <= max_sym; i++) { cum[i] = run; run = (uint16_t)(run + f[i]); }
    return 1;
}

/* EncSymbol (compress.rs:35-68) and the reciprocal update (:164-165) */
typedef struct { uint32_t freq, cmpl, bias, rcp, shift; } encsym_t;
static encsym_t encsym(uint32_t start, uint32_t freq) {
    encsym_t s;
    s.freq = freq; s.cmpl = RANS_PROB_SCALE - freq;
    if (freq < 2) { s.bias = start + RANS_PROB_SCALE - 1; s.rcp = 0xFFFFFFFFu; s.shift = 0; }
    else {
        uint32_t sh = 0;
        while (freq > (1u << sh)) sh++;
        s.rcp = (uint32_t)((((uint64_t)1 << (sh + 31)) + freq - 1) / freq);
        s.bias = start; s.shift = sh - 1;
    }
    return s;
}
static uint32_t encsym_update(const encsym_t *s, uint32_t x) {
    uint32_t q = (uint32_t)(((uint64_t)x * s->rcp) >> 32) >> s->shift;
    return x + s->bias + q * s->cmpl;
}
uint32_t por_rans_enc_update(uint32_t x, uint32_t start, uint32_t freq) {
    encsym_t s = encsym(start, freq);
    return encsym_update(&s, x);
}

/* compress.rs:187-260 */
int64_t por_rans_compress(uint8_t *dst, size_t cap, const uint8_t *src, size_t len, int *outcome) {
    *outcome = POR_OUT_INCOMPRESSIBLE;
    if (len == 0) return 0;
    uint32_t raw[256];
    por_histogram(src, len, raw);
    uint16_t f[256], cum[256];
    if (!por_rans_normalize(raw, f, cum)) return 0;
    encsym_t syms[256];
    for (int i = 0; i < 256; i++) syms[i] = encsym(cum[i], f[i]);
    /* encode_freq_table (compress.rs:128-135) */
    int max_sym = 0;
    for (int i = 0; i < 256; i++) if (f[i]) max_sym = i;
    size_t jt = 1 + 2 * (size_t)(max_sym + 1), header_len = jt + 16;
    if (header_len >= cap) { *outcome = POR_OUT_DST_TOO_SMALL; return 0; }
    dst[0] = (uint8_t)max_sym;
    for (int i = 0; i <= max_sym; i++) { dst[1 + 2 * i] = (uint8_t)f[i]; dst[2 + 2 * i] = (uint8_t)(f[i] >> 8); }
    memset(dst + jt, 0, 16);
    size_t s[4], e[4];
    por_split_four(len, s, e);
    size_t max_seg = 0;
    for (int i = 0; i < 4; i++) if (e[i] - s[i] > max_seg) max_seg = e[i] - s[i];
    size_t scap = 4 + 2 * max_seg + 16;
    uint8_t *scratch = (uint8_t *)malloc(scap);
    if (!scratch) return POR_ESMALL;
    uint32_t lens[4];
    size_t off = header_len;
    for (int i = 0; i < 4; i++) {
        /* encode_stream_into (compress.rs:140-185) */
        uint32_t x = RANS_L;
        size_t nb = 4;
        for (size_t k = e[i]; k > s[i]; k--) {
            const encsym_t *sy = &syms[src[k - 1]];
            uint32_t max_state = ((RANS_L >> RANS_PROB_BITS) << 8) * sy->freq;
            while (x >= max_state) {
                if (nb >= scap) { scap *= 2; scratch = (uint8_t *)realloc(scratch, scap); }
                scratch[nb++] = (uint8_t)(x & 0xFF);
                x >>= 8;
            }
            x = encsym_update(sy, x);
        }
        st32(scratch, x);
        for (size_t a = 4, b = nb - 1; a < b; a++, b--) { uint8_t t = scratch[a]; scratch[a] = scratch[b]; scratch[b] = t; }
        size_t written = nb;
        if (off + written > cap) { free(scratch); *outcome = POR_OUT_DST_TOO_SMALL; return 0; }
        if (written > 0xFFFFFFFFu) { free(scratch); *outcome = POR_OUT_LEN_OVERFLOW; return 0; }
        memcpy(dst + off, scratch, written);
        off += written;
        lens[i] = (uint32_t)written;
    }
    free(scratch);
    if (off >= len) { *outcome = POR_OUT_NOT_BENEFICIAL; return 0; }
    for (int i = 0; i < 4; i++) st32(dst + jt + 4 * i, lens[i]);
    *outcome = POR_OUT_ENCODED;
    return (int64_t)off;
}

/* decompress.rs:113-166 */
int64_t por_rans_decompress(uint8_t *dst, size_t dst_len, const uint8_t *src, size_t src_len) {
    /* decode_freq_table :24-52 */
    if (src_len == 0) return POR_EINVAL;
    size_t max_sym = src[0], need = 1 + 2 * (max_sym + 1);
    if (src_len < need) return POR_EINVAL;
    uint16_t f[256] = {0};
    uint32_t tot = 0;
    for (size_t i = 0; i <= max_sym; i++) { f[i] = (uint16_t)(src[1 + 2 * i] | (src[2 + 2 * i] << 8)); tot += f[i]; }
    if (tot != RANS_PROB_SCALE) return POR_EINVAL;
    size_t p = need;
    if (src_len - p < 16) return POR_EINVAL;
    uint64_t lens[4], total = 0;
    for (int i = 0; i < 4; i++) { lens[i] = ld32(src + p + 4 * i); total += lens[i]; }
    p += 16;
    if (total != (uint64_t)(src_len - p)) return POR_EINVAL;
    /* build_decode_table :55-77 */
    uint8_t tsym[RANS_PROB_SCALE];
    uint16_t tfreq[RANS_PROB_SCALE], tstart[RANS_PROB_SCALE];
    uint32_t pos = 0;
    for (int s = 0; s < 256; s++) {
        for (uint32_t j = 0; j < f[s]; j++) { tsym[pos + j] = (uint8_t)s; tfreq[pos + j] = f[s]; tstart[pos + j] = (uint16_t)pos; }
        pos += f[s];
    }
    size_t s[4], e[4];
    por_split_four(dst_len, s, e);
    size_t so = p;
    for (int i = 0; i < 4; i++) {
        const uint8_t *st = src + so;
        size_t sl = (size_t)lens[i];
        so += sl;
        if (s[i] == e[i]) continue;
        /* decode_stream :80-111 */
        if (sl < 4) return POR_EINVAL;
        uint32_t x = ld32(st);
        size_t q = 4;
        for (size_t k = s[i]; k < e[i]; k++) {
            uint32_t idx = x & (RANS_PROB_SCALE - 1);
            dst[k] = tsym[idx];
            x = (uint32_t)tfreq[idx] * (x >> RANS_PROB_BITS) + idx - tstart[idx];
            while (x < RANS_L) {
                if (q >= sl) return POR_EINVAL;
                x = (x << 8) | st[q++];
            }
        }
    }
    return (int64_t)dst_len;
}

/* ------------------------------------------------------------------------- */
/* tANS: entropy/tans/mod.rs (TABLE_LOG 11, single stream, LIFO bit stream)  */
/* ------------------------------------------------------------------------- */

#define TANS_LOG 11
#define TANS_L (1u << TANS_LOG)

static uint32_t highbit32(uint32_t x) { return 31u - (uint32_t)__builtin_clz(x); }

/* normalize :153-195 -- scale to sum L, every present symbol >= 1; surplus
 * comes off the first largest entry, deficit goes to the first most frequent
 * symbol */
static void tans_normalize(const uint32_t counts[256], uint64_t total, uint32_t norm[256]) {
    uint32_t sum = 0, max_count = 0;
    int max_sym = 0;
    for (int s = 0; s < 256; s++) {
        norm[s] = 0;
        if (!counts[s]) continue;
        uint32_t v = (uint32_t)(((uint64_t)counts[s] * TANS_L) / total);
        if (!v) v = 1;
        norm[s] = v;
        sum += v;
        if (counts[s] > max_count) { max_count = counts[s]; max_sym = s; }
    }
    while (sum > TANS_L) {
        int bi = -1;
        uint32_t bv = 1;
        for (int s = 0; s < 256; s++)
            if (norm[s] > bv) { bv = norm[s]; bi = s; }
        norm[bi]--;
        sum--;
    }
    while (sum < TANS_L) { norm[max_sym]++; sum++; }
}

/* spread :199-211 -- symbols in order, step (L/2 + L/8 + 3) mod L */
void por_tans_spread(const uint32_t norm[256], uint8_t table[2048]) {
    const uint32_t step = (TANS_L >> 1) + (TANS_L >> 3) + 3, mask = TANS_L - 1;
    uint32_t pos = 0;
    for (int s = 0; s < 256; s++)
        for (uint32_t k = 0; k < norm[s]; k++) { table[pos] = (uint8_t)s; pos = (pos + step) & mask; }
}

/* build_decode :346-368 -- slot u of symbol s with occurrence x (norm[s] ..
 * 2 norm[s] - 1): nb = 11 - floor(log2 x), baseline = (x << nb) - L */
void por_tans_decode_table(const uint32_t norm[256], uint8_t sym[2048], uint8_t nb[2048], uint16_t base[2048]) {
    uint32_t next[256];
    por_tans_spread(norm, sym);
    for (int s = 0; s < 256; s++) next[s] = norm[s];
    for (uint32_t u = 0; u < TANS_L; u++) {
        uint32_t x = next[sym[u]]++;
        uint32_t b = TANS_LOG - highbit32(x);
        nb[u] = (uint8_t)b;
        base[u] = (uint16_t)((x << b) - TANS_L);
    }
}

/* compress :273-341 -- returns the blob length, or 0 for "store raw" */
int64_t por_tans_compress(uint8_t *dst, size_t cap, const uint8_t *src, size_t n) {
    if (n == 0) return 0;
    uint32_t counts[256] = {0}, norm[256];
    for (size_t i = 0; i < n; i++) counts[src[i]]++;
    int nsym = 0;
    for (int s = 0; s < 256; s++) nsym += counts[s] != 0;
    if (nsym < 2) return 0;
    tans_normalize(counts, n, norm);
    uint8_t sym[TANS_L];
    por_tans_spread(norm, sym);
    /* build_encode :225-268: next-state table packed per symbol and the
     * per-symbol (delta_nb_bits, delta_find_state) transform */
    uint32_t cumul[256], fill[256], run = 0;
    for (int s = 0; s < 256; s++) { cumul[s] = run; run += norm[s]; fill[s] = cumul[s]; }
    uint16_t state_table[TANS_L];
    for (uint32_t u = 0; u < TANS_L; u++) state_table[fill[sym[u]]++] = (uint16_t)(TANS_L + u);
    uint32_t dnb[256] = {0};
    int32_t dfs[256] = {0};
    int32_t total = 0;
    for (int s = 0; s < 256; s++) {
        uint32_t c = norm[s];
        if (!c) continue;
        if (c == 1) {
            dnb[s] = (TANS_LOG << 16) - TANS_L;
            dfs[s] = total - 1;
            total += 1;
        } else {
            uint32_t max_bits = TANS_LOG - highbit32(c - 1);
            dnb[s] = (max_bits << 16) - (c << max_bits);
            dfs[s] = total - (int32_t)c;
            total += (int32_t)c;
        }
    }
    /* LSB-first bit writer :60-100; symbols encoded last to first from state L */
    size_t bs_cap = n * 2 + 16;
    uint8_t *bs = (uint8_t *)malloc(bs_cap);
    if (!bs) return POR_ESMALL;
    size_t bl = 0;
    uint64_t acc = 0, tot = 0;
    uint32_t nbits = 0, value = TANS_L;
    for (size_t i = n; i-- > 0;) {
        uint8_t b = src[i];
        uint32_t k = (value + dnb[b]) >> 16;
        if (k) {
            acc |= ((uint64_t)value & ((1ull << k) - 1)) << nbits;
            nbits += k; tot += k;
            while (nbits >= 8) { bs[bl++] = (uint8_t)acc; acc >>= 8; nbits -= 8; }
        }
        value = state_table[(int32_t)(value >> k) + dfs[b]];
    }
    acc |= ((uint64_t)value & (TANS_L - 1)) << nbits;
    nbits += TANS_LOG; tot += TANS_LOG;
    while (nbits >= 8) { bs[bl++] = (uint8_t)acc; acc >>= 8; nbits -= 8; }
    if (nbits) bs[bl++] = (uint8_t)acc;
    size_t blob = 1 + 2 + (size_t)nsym * 3 + 8 + bl;
    if (blob >= n || blob > cap) { free(bs); return 0; }
    size_t w = 0;
    dst[w++] = TANS_LOG;
    dst[w++] = (uint8_t)nsym; dst[w++] = (uint8_t)(nsym >> 8);
    for (int s = 0; s < 256; s++) {
        if (!norm[s]) continue;
        dst[w++] = (uint8_t)s; dst[w++] = (uint8_t)norm[s]; dst[w++] = (uint8_t)(norm[s] >> 8);
    }
    st32(dst + w, (uint32_t)tot); st32(dst + w + 4, (uint32_t)(tot >> 32)); w += 8;
    memcpy(dst + w, bs, bl);
    free(bs);
    return (int64_t)(w + bl);
}

/* LIFO reader :102-150: pops the nb most recently written bits */
static int tans_read(const uint8_t *bs, size_t bl, uint64_t *pos, uint32_t nb, uint32_t *v) {
    if (nb == 0) { *v = 0; return 0; }
    if (*pos < nb) return -1;
    uint64_t start = *pos - nb;
    size_t bi = (size_t)(start >> 3);
    uint32_t w = bs[bi];
    if (bi + 1 < bl) w |= (uint32_t)bs[bi + 1] << 8;
    if (bi + 2 < bl) w |= (uint32_t)bs[bi + 2] << 16;
    *v = (w >> (start & 7)) & ((1u << nb) - 1);
    *pos = start;
    return 0;
}

/* decompress :372-455 -- n symbols from a compress blob */
int64_t por_tans_decompress(uint8_t *dst, size_t n, const uint8_t *src, size_t len) {
    if (n == 0) return 0;
    if (len < 3) return POR_EINVAL;
    if (src[0] != TANS_LOG) return POR_EINVAL;
    size_t nsym = (size_t)src[1] | ((size_t)src[2] << 8);
    if (nsym < 2 || nsym > 256) return POR_EINVAL;
    size_t p = 3, pairs_end = p + nsym * 3;
    if (pairs_end + 8 > len) return POR_EINVAL;
    uint32_t norm[256] = {0}, sum = 0;
    for (size_t i = 0; i < nsym; i++, p += 3) {
        uint32_t s = src[p], f = (uint32_t)src[p + 1] | ((uint32_t)src[p + 2] << 8);
        if (norm[s]) return POR_EINVAL;        /* duplicate symbol */
        if (!f) return POR_EINVAL;             /* zero frequency */
        norm[s] = f;
        sum += f;
    }
    if (sum != TANS_L) return POR_EINVAL;
    uint64_t total_bits = ld64(src + p);
    p += 8;
    const uint8_t *bs = src + p;
    size_t bl = len - p;
    if (total_bits > (uint64_t)bl * 8) return POR_EINVAL;
    uint8_t sym[TANS_L], nb[TANS_L];
    uint16_t base[TANS_L];
    por_tans_decode_table(norm, sym, nb, base);
    uint64_t pos = total_bits;
    uint32_t state, low;
    if (tans_read(bs, bl, &pos, TANS_LOG, &state)) return POR_EINVAL;
    if (state >= TANS_L) return POR_EINVAL;
    for (size_t i = 0; i < n; i++) {
        dst[i] = sym[state];
        if (tans_read(bs, bl, &pos, nb[state], &low)) return POR_EINVAL;
        state = base[state] + low;
        if (state >= TANS_L) return POR_EINVAL;
    }
    if (pos != 0) return POR_EINVAL;           /* trailing bits */
    if (state != 0) return POR_EINVAL;         /* not back at the start state */
    return (int64_t)n;
}

/* ------------------------------------------------------------------------- */
/* plane codec payloads: codecs/huffman.rs:37-141, codecs/rans.rs:38-144,    */
/* codec_tagged.rs:98-194, codecs/length_prefix.rs:30-33, codecs/identity.rs  */
/* ------------------------------------------------------------------------- */

size_t por_codec_encode_bound(size_t len) { return len + 5; }

static int length_prefix_accepted(size_t decoded_len, size_t body_len) {
    if (decoded_len > 0xFFFFFFFFu) return 0;
    return decoded_len <= ((size_t)1 << 30) || decoded_len <= body_len * 64;
}

static int64_t emit_raw(const uint8_t *plane, size_t len, uint8_t *out, size_t cap) {
    if (1 + len > cap) return POR_ESMALL;
    out[0] = 0;
    if (len) memcpy(out + 1, plane, len);
    return (int64_t)(1 + len);
}

int64_t por_codec_encode(int codec, const uint8_t *plane, size_t len, uint8_t *out, size_t cap) {
    if (codec == POR_CODEC_IDENTITY) {
        if (len > cap) return POR_ESMALL;
        if (len) memcpy(out, plane, len);
        return (int64_t)len;
    }
    if (codec != POR_CODEC_HUFFMAN && codec != POR_CODEC_RANS && codec != POR_CODEC_TANS) return POR_EUNSUP;
    if (len == 0) { if (cap < 1) return POR_ESMALL; out[0] = 0; return 1; }
    size_t bound = len * 2 + 4096;          /* huffman_output_bound / rans_output_bound */
    uint8_t *buf = (uint8_t *)malloc(bound);
    if (!buf) return POR_ESMALL;
    int outcome;
    int64_t n;
    if (codec == POR_CODEC_TANS) {          /* codecs/tans.rs:39-92: scratch of plane.len() bytes */
        n = por_tans_compress(buf, len, plane, len);
        outcome = n > 0 ? POR_OUT_ENCODED : POR_OUT_NOT_BENEFICIAL;
    } else
        n = codec == POR_CODEC_HUFFMAN ? por_huf_compress(buf, bound, plane, len, &outcome)
                                       : por_rans_compress(buf, bound, plane, len, &outcome);
    int64_t r;
    if (n < 0) r = n;
    else if (outcome == POR_OUT_ENCODED && len <= 0xFFFFFFFFu &&
             (codec == POR_CODEC_HUFFMAN || length_prefix_accepted(len, (size_t)n))) {
        if ((size_t)n + 5 > cap) r = POR_ESMALL;
        else {
            out[0] = 1; st32(out + 1, (uint32_t)len);
            memcpy(out + 5, buf, (size_t)n);
            r = n + 5;
        }
    } else r = emit_raw(plane, len, out, cap);
    free(buf);
    return r;
}

int64_t por_codec_decoded_len(int codec, const uint8_t *payload, size_t len) {
    if (codec == POR_CODEC_IDENTITY) return (int64_t)len;
    if (len == 0) return POR_EINVAL;
    if (payload[0] == 0) return (int64_t)(len - 1);
    if (payload[0] != 1 || len < 5) return POR_EINVAL;
    return (int64_t)ld32(payload + 1);
}

int64_t por_codec_decode(int codec, const uint8_t *pl, size_t len, uint8_t *out, size_t cap) {
    if (codec == POR_CODEC_IDENTITY) {            /* identity.rs decode + check_decoded_len */
        if (len > cap) return POR_EINVAL;
        if (len) memcpy(out, pl, len);
        return (int64_t)len;
    }
    if (codec == POR_CODEC_ZSTD) {                /* zstd.rs decode_bounded: the payload is the frames */
        int64_t n = por_zstd_decompress(out, cap, pl, len);
        return n < 0 ? POR_EINVAL : n;
    }
    if (codec != POR_CODEC_HUFFMAN && codec != POR_CODEC_RANS && codec != POR_CODEC_TANS) return POR_EUNSUP;
    if (len == 0) return POR_EINVAL;
    uint8_t tag = pl[0];
    if (tag == 0) {
        if (len - 1 > cap) return POR_EINVAL;
        if (len > 1) memcpy(out, pl + 1, len - 1);
        return (int64_t)(len - 1);
    }
    if (tag != 1) return POR_EINVAL;
    if (len - 1 < 4) return POR_EINVAL;
    size_t orig = ld32(pl + 1);
    const uint8_t *enc = pl + 5;
    size_t enc_len = len - 5;
    if (codec == POR_CODEC_HUFFMAN) {
        if (orig > enc_len * 32 + 4096) return POR_EINVAL;   /* huffman.rs:122-131 */
        if (orig > cap) return POR_EINVAL;                    /* check_decoded_len */
        return por_huf_decompress(out, orig, enc, enc_len);
    }
    /* rANS / tANS: decode_bounded's check_within runs first (rans.rs:158-160,
     * tans.rs:150-152), then the length-prefix rule (tans.rs:118-126) */
    if (orig > cap) return POR_EINVAL;
    if (!length_prefix_accepted(orig, enc_len)) return POR_EINVAL;
    if (orig == 0) return 0;                                  /* decode_tagged expected_len == 0 */
    if (codec == POR_CODEC_TANS) return por_tans_decompress(out, orig, enc, enc_len);
    return por_rans_decompress(out, orig, enc, enc_len);
}

/* ------------------------------------------------------------------------- */
/* trial-encode selection: select.rs:27-64 over a menu in dispatch.rs:13-49   */
/* order; the smallest state + payload wins, the first in the menu on ties    */
/* ------------------------------------------------------------------------- */

int64_t por_select_encode(const uint8_t *plane, size_t len, const uint16_t *menu, size_t menu_len,
                          uint16_t *chosen, uint8_t *out, size_t cap) {
    if (menu_len == 0) return POR_EINVAL;                 /* "empty codec menu" */
    size_t bound = por_codec_encode_bound(len);
    uint8_t *tmp = (uint8_t *)malloc(bound ? bound : 1);
    if (!tmp) return POR_ESMALL;
    int64_t best = -1;
    for (size_t i = 0; i < menu_len; i++) {
        int64_t n = por_codec_encode(menu[i], plane, len, tmp, bound);
        if (n < 0) { free(tmp); return n; }
        if (best < 0 || n < best) {                       /* min_by_key keeps the first minimum */
            if ((size_t)n > cap) { free(tmp); return POR_ESMALL; }
            best = n;
            *chosen = menu[i];
            memcpy(out, tmp, (size_t)n);
        }
    }
    free(tmp);
    return best;
}

/* ------------------------------------------------------------------------- */
/* chunk framing: compressor.rs:316-381, container.rs:1975-2050               */
/* ------------------------------------------------------------------------- */

int64_t por_encode_plane_chunked(int codec, const uint8_t *plane, size_t len, uint32_t chunk_size,
                                 uint8_t *out, size_t cap, uint32_t *ent, size_t max_ent, size_t *n_chunks) {
    size_t cs = chunk_size ? chunk_size : 1;
    size_t nch = len == 0 ? 1 : (len + cs - 1) / cs;
    if (nch > max_ent) return POR_ESMALL;
    size_t off = 0;
    for (size_t k = 0; k < nch; k++) {
        size_t a = k * cs, b = a + cs > len ? len : a + cs;
        if (off > 0xFFFFFFFFu) return POR_EINVAL;
        if (off + 5 > cap) return POR_ESMALL;
        out[off] = 0; st32(out + off + 1, 0);      /* frame_chunk: [ver=0][state_len=0] */
        int64_t n = por_codec_encode(codec, plane + a, b - a, out + off + 5, cap - off - 5);
        if (n < 0) return n;
        ent[2 * k] = (uint32_t)off; ent[2 * k + 1] = (uint32_t)(b - a);
        off += 5 + (size_t)n;
    }
    *n_chunks = nch;
    return (int64_t)off;
}

static int64_t decode_one_chunk(int codec, const uint8_t *payload, size_t payload_len, const uint32_t *ent,
                                size_t n_chunks, size_t i, uint8_t *dst) {
    size_t start = ent[2 * i], end = i + 1 < n_chunks ? ent[2 * (i + 1)] : payload_len;
    if (start > end || end > payload_len) return POR_EINVAL;
    const uint8_t *fr = payload + start;
    size_t fl = end - start;
    if (fl < 5) return POR_EINVAL;
    size_t sl = ld32(fr + 1);
    if (fl - 5 < sl) return POR_EINVAL;
    size_t want = ent[2 * i + 1];
    int64_t n = por_codec_decode(codec, fr + 5 + sl, fl - 5 - sl, dst, want);
    if (n < 0) return n;
    if ((size_t)n != want) return POR_EINVAL;
    return n;
}

int64_t por_decode_plane_chunked(int codec, const uint8_t *payload, size_t payload_len, const uint32_t *ent,
                                 size_t n_chunks, uint8_t *out, size_t cap) {
    size_t total = 0;
    for (size_t i = 0; i < n_chunks; i++) total += ent[2 * i + 1];
    if (total > cap) return POR_EINVAL;
    size_t o = 0;
    for (size_t i = 0; i < n_chunks; i++) {
        int64_t n = decode_one_chunk(codec, payload, payload_len, ent, n_chunks, i, out + o);
        if (n < 0) return n;
        o += (size_t)n;
    }
    return (int64_t)o;
}

typedef struct {
    int codec; const uint8_t *payload; size_t payload_len; const uint32_t *ent; size_t n;
    const size_t *dst_off; uint8_t *out; size_t next; pthread_mutex_t *mu; int64_t err;
} mt_job_t;

static void *mt_worker(void *arg) {
    mt_job_t *j = (mt_job_t *)arg;
    for (;;) {
        pthread_mutex_lock(j->mu);
        size_t i = j->next++;
        pthread_mutex_unlock(j->mu);
        if (i >= j->n) break;
        int64_t r = decode_one_chunk(j->codec, j->payload, j->payload_len, j->ent, j->n, i, j->out + j->dst_off[i]);
        if (r < 0) { pthread_mutex_lock(j->mu); j->err = r; pthread_mutex_unlock(j->mu); }
    }
    return NULL;
}

int64_t por_decode_plane_chunked_mt(int codec, const uint8_t *payload, size_t payload_len, const uint32_t *ent,
                                    size_t n_chunks, uint8_t *out, size_t cap, int threads) {
    if (threads <= 1) return por_decode_plane_chunked(codec, payload, payload_len, ent, n_chunks, out, cap);
    size_t *dst_off = (size_t *)malloc((n_chunks + 1) * sizeof(size_t));
    if (!dst_off) return POR_ESMALL;
    size_t total = 0;
    for (size_t i = 0; i < n_chunks; i++) { dst_off[i] = total; total += ent[2 * i + 1]; }
    if (total > cap) { free(dst_off); return POR_EINVAL; }
    pthread_mutex_t mu = PTHREAD_MUTEX_INITIALIZER;
    mt_job_t job = {codec, payload, payload_len, ent, n_chunks, dst_off, out, 0, &mu, 0};
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
    for (int t = 0; t < threads; t++) pthread_create(&th[t], NULL, mt_worker, &job);
    for (int t = 0; t < threads; t++) pthread_join(th[t], NULL);
    free(th); free(dst_off);
    return job.err ? job.err : (int64_t)total;
}

/* Whole-container decode, the timed CPU baseline: tensors in parallel over
 * `threads` pthreads (container.rs:1766-1780 runs the per-tensor decode over
 * rayon workers), each tensor's planes chunk by chunk (container.rs:
 * 1975-2050) into per-worker plane buffers, then the fused inverse chain
 * into the tensor's output (fusion.rs inverse, via por_chain_inverse).
 * Tensor t has planes np = por_chain_nplanes(chain); plane p of tensor t is
 * payloads[t * np + p] (payload_lens, entries, n_entries likewise), plane
 * length out_lens[t] / ratio.  Returns 0 or the first error. */
typedef struct {
    int codec, chain, np; size_t n;
    const uint8_t *const *payloads; const size_t *payload_lens;
    const uint32_t *const *entries; const size_t *n_entries;
    uint8_t *const *outs; const size_t *out_lens;
    size_t next, max_plane; pthread_mutex_t *mu; int64_t err;
} mtt_job_t;

static void *mtt_worker(void *arg) {
    mtt_job_t *j = (mtt_job_t *)arg;
    uint8_t *buf[4] = {0, 0, 0, 0};
    for (int p = 0; p < j->np; p++) buf[p] = (uint8_t *)malloc(j->max_plane ? j->max_plane : 1);
    for (;;) {
        pthread_mutex_lock(j->mu);
        size_t t = j->next++;
        pthread_mutex_unlock(j->mu);
        if (t >= j->n) break;
        int64_t plane_len = por_chain_plane_len(j->chain, j->out_lens[t]);
        int64_t r = plane_len < 0 ? POR_EINVAL : 0;
        for (int p = 0; p < j->np && r >= 0; p++) {
            size_t k = t * (size_t)j->np + (size_t)p;
            r = por_decode_plane_chunked(j->codec, j->payloads[k], j->payload_lens[k], j->entries[k],
                                         j->n_entries[k], buf[p], (size_t)plane_len);
            if (r >= 0 && r != plane_len) r = POR_EINVAL;
        }
        if (r >= 0) r = por_chain_inverse(j->chain, (const uint8_t *const *)buf, (size_t)plane_len, j->outs[t]);
        if (r < 0) { pthread_mutex_lock(j->mu); j->err = r; pthread_mutex_unlock(j->mu); }
    }
    for (int p = 0; p < j->np; p++) free(buf[p]);
    return NULL;
}

int64_t por_decode_tensors_mt(int codec, int chain, size_t n_tensors, const uint8_t *const *payloads,
                              const size_t *payload_lens, const uint32_t *const *entries, const size_t *n_entries,
                              uint8_t *const *outs, const size_t *out_lens, int threads) {
    int np = por_chain_nplanes(chain);
    if (np <= 0 || np > 4) return POR_EINVAL;
    size_t max_plane = 0;
    for (size_t t = 0; t < n_tensors; t++) {
        int64_t pl = por_chain_plane_len(chain, out_lens[t]);
        if (pl < 0) return POR_EINVAL;
        if ((size_t)pl > max_plane) max_plane = (size_t)pl;
    }
    if (threads < 1) threads = 1;
    pthread_mutex_t mu = PTHREAD_MUTEX_INITIALIZER;
    mtt_job_t job = {codec, chain, np, n_tensors, payloads, payload_lens, entries, n_entries,
                     outs, out_lens, 0, max_plane, &mu, 0};
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
    for (int t = 0; t < threads; t++) pthread_create(&th[t], NULL, mtt_worker, &job);
    for (int t = 0; t < threads; t++) pthread_join(th[t], NULL);
    free(th);
    return job.err;
}

/* ------------------------------------------------------------------------- */
/* Per-config CPU baselines: a batch of tensors of any chain, each plane with */
/* its own codec, chunked (chunk frames + table, compressor.rs:316-381) or    */
/* not.  Decode: every chunk of every plane of every tensor is one unit on a  */
/* shared queue over `threads` pthreads (container.rs:1773 runs tensors and   */
/* :1996 their chunks on rayon workers), then each tensor's inverse chain in  */
/* slices of 2^20 plane positions over the same workers (the reference runs   */
/* a tensor's inverse on one worker: slicing only helps the CPU figure).      */
/* Encode: the forward chain in slices, then one unit per chunk (written at a */
/* fixed stride), then each plane's frames packed together with its table.   */
/* ------------------------------------------------------------------------- */

#define BATCH_SLICE ((size_t)1 << 20)

typedef struct { size_t plane, chunk, dst, len; } batch_unit_t;
typedef struct { size_t tensor, a, b; } batch_slice_t;

typedef struct {
    size_t n_units, n_slices, n_planes;
    batch_unit_t *units; batch_slice_t *slices;
    const int *chains; const size_t *plane_base;
    /* decode */
    const size_t *out_lens; uint8_t *const *outs;
    const int *codecs; const uint8_t *const *payloads; const size_t *payload_lens;
    const uint32_t *const *entries; const size_t *n_entries;
    uint8_t *const *plane_bufs;
    /* encode */
    const uint8_t *const *ins; const uint32_t *chunk_sizes; uint8_t *const *enc_outs;
    uint32_t *const *enc_entries; size_t *enc_lens; size_t *unit_len;
    size_t next_unit, next_slice, next_plane;
    pthread_barrier_t bar;
    int64_t err;
} batch_job_t;

static void batch_fail(batch_job_t *j, int64_t r) { __atomic_store_n(&j->err, r, __ATOMIC_RELAXED); }

static size_t batch_out_per_pos(int chain) {
    return chain == POR_CHAIN_IEEE16_SPLIT2 ? 2 : chain == POR_CHAIN_IEEE32_SPLIT4 ? 4 : 1;
}

static void *batch_decode_worker(void *arg) {
    batch_job_t *j = (batch_job_t *)arg;
    for (;;) {
        size_t u = __atomic_fetch_add(&j->next_unit, 1, __ATOMIC_RELAXED);
        if (u >= j->n_units) break;
        const batch_unit_t *U = &j->units[u];
        size_t k = U->plane;
        int64_t r;
        if (j->n_entries[k] == 0) {
            r = por_codec_decode(j->codecs[k], j->payloads[k], j->payload_lens[k], j->plane_bufs[k], U->dst);
            if (r >= 0 && (size_t)r != U->dst) r = POR_EINVAL;
        } else {
            r = decode_one_chunk(j->codecs[k], j->payloads[k], j->payload_lens[k], j->entries[k], j->n_entries[k],
                                 U->chunk, j->plane_bufs[k] + U->dst);
        }
        if (r < 0) batch_fail(j, r);
    }
    pthread_barrier_wait(&j->bar);
    for (;;) {
        size_t s = __atomic_fetch_add(&j->next_slice, 1, __ATOMIC_RELAXED);
        if (s >= j->n_slices || __atomic_load_n(&j->err, __ATOMIC_RELAXED)) break;
        const batch_slice_t *S = &j->slices[s];
        int chain = j->chains[S->tensor];
        size_t base = j->plane_base[S->tensor];
        const uint8_t *pl[4] = {0, 0, 0, 0};
        for (int p = 0; p < por_chain_nplanes(chain); p++) pl[p] = j->plane_bufs[base + p] + S->a;
        int r = por_chain_inverse(chain, pl, S->b - S->a, j->outs[S->tensor] + S->a * batch_out_per_pos(chain));
        if (r < 0) batch_fail(j, r);
    }
    return NULL;
}

/* Plans the units and slices shared by both directions; plane lengths from
 * the tensor lengths.  Returns 0 or an error. */
static int64_t batch_plan(batch_job_t *j, size_t n_tensors, const size_t *lens, int decode) {
    size_t np_total = 0, n_units = 0, n_slices = 0;
    size_t *base = (size_t *)malloc((n_tensors + 1) * sizeof(size_t));
    if (!base) return POR_ESMALL;
    for (size_t t = 0; t < n_tensors; t++) {
        int np = por_chain_nplanes(j->chains[t]);
        int64_t pl = por_chain_plane_len(j->chains[t], lens[t]);
        if (np <= 0 || pl < 0) { free(base); return POR_EINVAL; }
        base[t] = np_total;
        for (int p = 0; p < np; p++) {
            size_t k = np_total + (size_t)p;
            if (decode) n_units += j->n_entries[k] ? j->n_entries[k] : 1;
            else n_units += j->chunk_sizes[k] ? ((size_t)pl + j->chunk_sizes[k] - 1) / j->chunk_sizes[k] + !pl : 1;
        }
        np_total += (size_t)np;
        n_slices += ((size_t)pl + BATCH_SLICE - 1) / BATCH_SLICE;
    }
    base[n_tensors] = np_total;
    j->units = (batch_unit_t *)malloc((n_units + 1) * sizeof(batch_unit_t));
    j->slices = (batch_slice_t *)malloc((n_slices + 1) * sizeof(batch_slice_t));
    if (!j->units || !j->slices) { free(base); return POR_ESMALL; }
    size_t u = 0, s = 0;
    for (size_t t = 0; t < n_tensors; t++) {
        size_t pl = (size_t)por_chain_plane_len(j->chains[t], lens[t]);
        for (size_t k = base[t]; k < base[t + 1]; k++) {
            if (decode && j->n_entries[k]) {
                size_t dst = 0;
                for (size_t i = 0; i < j->n_entries[k]; i++) {
                    j->units[u++] = (batch_unit_t){k, i, dst, j->entries[k][2 * i + 1]};
                    dst += j->entries[k][2 * i + 1];
                }
                if (dst != pl) { free(base); return POR_EINVAL; }
            } else if (!decode && j->chunk_sizes[k]) {
                size_t cs = j->chunk_sizes[k], nch = pl ? (pl + cs - 1) / cs : 1;
                for (size_t i = 0; i < nch; i++)
                    j->units[u++] = (batch_unit_t){k, i, i * cs, (i + 1) * cs < pl ? cs : pl - i * cs};
            } else {
                j->units[u++] = (batch_unit_t){k, (size_t)-1, pl, pl};
            }
        }
        for (size_t a = 0; a < pl; a += BATCH_SLICE)
            j->slices[s++] = (batch_slice_t){t, a, a + BATCH_SLICE < pl ? a + BATCH_SLICE : pl};
    }
    j->n_units = u;
    j->n_slices = s;
    j->n_planes = np_total;
    j->plane_base = base;
    return 0;
}

static void batch_free(batch_job_t *j) {
    free(j->units);
    free(j->slices);
    free((void *)j->plane_base);
}

static int64_t batch_run(batch_job_t *j, int threads, void *(*fn)(void *)) {
    if (threads < 1) threads = 1;
    pthread_barrier_init(&j->bar, NULL, (unsigned)threads);
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
    if (!th) return POR_ESMALL;
    for (int t = 0; t < threads; t++) pthread_create(&th[t], NULL, fn, j);
    for (int t = 0; t < threads; t++) pthread_join(th[t], NULL);
    free(th);
    pthread_barrier_destroy(&j->bar);
    return j->err;
}

int64_t por_batch_decode_mt(size_t n_tensors, const int *chains, const size_t *out_lens, uint8_t *const *outs,
                            const int *codecs, const uint8_t *const *payloads, const size_t *payload_lens,
                            const uint32_t *const *entries, const size_t *n_entries, uint8_t *const *plane_bufs,
                            int threads) {
    batch_job_t j;
    memset(&j, 0, sizeof j);
    j.chains = chains; j.out_lens = out_lens; j.outs = outs; j.codecs = codecs; j.payloads = payloads;
    j.payload_lens = payload_lens; j.entries = entries; j.n_entries = n_entries; j.plane_bufs = plane_bufs;
    int64_t r = batch_plan(&j, n_tensors, out_lens, 1);
    if (r == 0) r = batch_run(&j, threads, batch_decode_worker);
    batch_free(&j);
    return r;
}

static void *batch_encode_worker(void *arg) {
    batch_job_t *j = (batch_job_t *)arg;
    for (;;) {   /* forward chain, slice by slice, into the plane buffers */
        size_t s = __atomic_fetch_add(&j->next_slice, 1, __ATOMIC_RELAXED);
        if (s >= j->n_slices) break;
        const batch_slice_t *S = &j->slices[s];
        int chain = j->chains[S->tensor];
        size_t base = j->plane_base[S->tensor];
        uint8_t *pl[4] = {0, 0, 0, 0};
        for (int p = 0; p < por_chain_nplanes(chain); p++) pl[p] = j->plane_bufs[base + p] + S->a;
        size_t w = batch_out_per_pos(chain);
        int r = por_chain_forward(chain, j->ins[S->tensor] + S->a * w, (S->b - S->a) * w, pl);
        if (r < 0) batch_fail(j, r);
    }
    pthread_barrier_wait(&j->bar);
    for (;;) {   /* one chunk (or unchunked plane) per unit, at its fixed stride */
        size_t u = __atomic_fetch_add(&j->next_unit, 1, __ATOMIC_RELAXED);
        if (u >= j->n_units || __atomic_load_n(&j->err, __ATOMIC_RELAXED)) break;
        const batch_unit_t *U = &j->units[u];
        size_t k = U->plane;
        int64_t n;
        if (U->chunk == (size_t)-1) {
            n = por_codec_encode(j->codecs[k], j->plane_bufs[k], U->dst, j->enc_outs[k], por_codec_encode_bound(U->dst));
        } else {
            size_t cs = j->chunk_sizes[k], len = U->len;
            uint8_t *o = j->enc_outs[k] + U->chunk * (5 + por_codec_encode_bound(cs));
            o[0] = 0; st32(o + 1, 0);
            n = por_codec_encode(j->codecs[k], j->plane_bufs[k] + U->dst, len, o + 5, por_codec_encode_bound(cs));
            if (n >= 0) n += 5;
        }
        if (n < 0) batch_fail(j, n);
        else j->unit_len[u] = (size_t)n;
    }
    pthread_barrier_wait(&j->bar);
    for (;;) {   /* pack each chunked plane's frames and write its table */
        size_t k = __atomic_fetch_add(&j->next_plane, 1, __ATOMIC_RELAXED);
        if (k >= j->n_planes || __atomic_load_n(&j->err, __ATOMIC_RELAXED)) break;
        size_t off = 0, i = 0;
        for (size_t u = 0; u < j->n_units; u++) {
            if (j->units[u].plane != k) continue;
            if (j->units[u].chunk == (size_t)-1) { off = j->unit_len[u]; break; }
            size_t stride = 5 + por_codec_encode_bound(j->chunk_sizes[k]);
            memmove(j->enc_outs[k] + off, j->enc_outs[k] + i * stride, j->unit_len[u]);
            j->enc_entries[k][2 * i] = (uint32_t)off;
            j->enc_entries[k][2 * i + 1] = (uint32_t)j->units[u].len;
            off += j->unit_len[u];
            i++;
        }
        j->enc_lens[k] = off;
    }
    return NULL;
}

/* Encode batch: enc_outs[k] must hold n_chunks * (5 + bound(chunk)) bytes
 * (one codec bound of the plane when unchunked), enc_entries[k] 2 u32 per
 * chunk; enc_lens[k] receives the packed payload length. */
int64_t por_batch_encode_mt(size_t n_tensors, const int *chains, const size_t *in_lens, const uint8_t *const *ins,
                            const int *codecs, const uint32_t *chunk_sizes, uint8_t *const *plane_bufs,
                            uint8_t *const *enc_outs, uint32_t *const *enc_entries, size_t *enc_lens, int threads) {
    batch_job_t j;
    memset(&j, 0, sizeof j);
    j.chains = chains; j.ins = ins; j.codecs = codecs; j.chunk_sizes = chunk_sizes; j.plane_bufs = plane_bufs;
    j.enc_outs = enc_outs; j.enc_entries = enc_entries; j.enc_lens = enc_lens;
    int64_t r = batch_plan(&j, n_tensors, in_lens, 0);
    if (r == 0) {
        j.unit_len = (size_t *)calloc(j.n_units + 1, sizeof(size_t));
        if (!j.unit_len) r = POR_ESMALL;
    }
    if (r == 0) r = batch_run(&j, threads, batch_encode_worker);
    free(j.unit_len);
    batch_free(&j);
    return r;
}

/* ------------------------------------------------------------------------- */
/* huff_ilv (this build's own codec; executable specification)               */
/*                                                                           */
/* payload: [tag u8] tag 0: stored plane bytes follow.  tag 2: packed       */
/*   nibbles (ilv_emit_packed).  tag 1:                                      */
/*   [orig_len u32][weights header (weights.rs)][0-pad to 4][off u32 x nb+1] */
/*   [data]; nb = ceil(n / 16384).  Block b = data[off[b]..off[b+1]):        */
/*   [64 x u8 lane word counts][lane 0 words][lane 1 words]...(u32 LE).      */
/*   Lane j codes groups g = j + 64 r (r = 0..15), group g = plane positions  */
/*   [b*16384 + 16 g, +16) clipped to n, as rev(canonical code) bits packed  */
/*   LSB-first into its words (the reference's code/bit order, tree.rs).     */
/* Code lengths: the reference tree (tree.rs:19-85) with its length limit    */
/*   (tree.rs:212-242) set to 6 when every symbol is < 16 (nibble planes),   */
/*   else 11.  Any lengths <= 11 decode; <= 6 lets decoders take two         */
/*   symbols per 12-bit table lookup.                                        */
/* ------------------------------------------------------------------------- */

#define ILV_BLOCK 16384

/* Packed nibbles, the third payload form of both GPU-native codecs: a plane
 * whose symbols are all < 16 may be stored two symbols per byte:
 *   [0x02][n u32][0 0 0][ceil(n / 2) bytes], byte i = s[2i] | s[2i+1] << 4
 * (the high nibble of the last byte is 0 when n is odd).  Encoders choose
 * the smallest of coded, packed and stored (packed needs n >= 16 to beat
 * stored; coded wins only when strictly smaller than both). */
static size_t ilv_packed_size(size_t n) { return 8 + (n + 1) / 2; }

static int ilv_all_nibbles(const uint32_t freqs[256]) {
    for (int s = 16; s < 256; s++) if (freqs[s]) return 0;
    return 1;
}

static int64_t ilv_emit_packed(const uint8_t *plane, size_t n, uint8_t *out, size_t cap) {
    size_t len = ilv_packed_size(n);
    if (len > cap) return POR_ESMALL;
    memset(out, 0, len);
    out[0] = 2; st32(out + 1, (uint32_t)n);
    for (size_t i = 0; i < n; i++) out[8 + i / 2] |= (uint8_t)((plane[i] & 0xF) << (4 * (i & 1)));
    return (int64_t)len;
}

static int64_t ilv_decode_packed(const uint8_t *p, size_t len, uint8_t *out, size_t cap) {
    if (len < 8 || p[5] || p[6] || p[7]) return POR_EINVAL;
    size_t n = ld32(p + 1);
    if (len != ilv_packed_size(n)) return POR_EINVAL;
    if ((n & 1) && (p[len - 1] >> 4)) return POR_EINVAL;
    if (n > cap) return POR_ESMALL;
    for (size_t i = 0; i < n; i++) out[i] = (uint8_t)((p[8 + i / 2] >> (4 * (i & 1))) & 0xF);
    return (int64_t)n;
}
#define ILV_LANES 64
#define ILV_GROUP 16
#define ILV_NIBBLE_MAX_LEN 6

/* the huff_ilv encoder's code lengths (see above) */
int por_ilv_lengths(const uint32_t freqs[256], uint8_t lengths[256]) {
    int nibble = 1;
    for (int s = 16; s < 256; s++) if (freqs[s]) nibble = 0;
    return por_huf_lengths_limited(freqs, lengths, nibble ? ILV_NIBBLE_MAX_LEN : HUF_MAX_TABLE_LOG);
}

size_t por_ilv_encode_bound(size_t len) {
    size_t nb = (len + ILV_BLOCK - 1) / ILV_BLOCK;
    return 1 + len + 5 + 130 + 3 + 4 * (nb + 1) + nb * 64 + len * 11 / 8 + nb * 64 * 4 + 16;
}

/* force_coded: the coded form (tag 1) whatever its size, POR_EINVAL when the
 * plane has no code (empty); test fixtures only (decoders must accept any
 * valid coded payload, also one no encoder would choose). */
static int64_t ilv_encode_impl(const uint8_t *plane, size_t n, uint8_t *out, size_t cap, int force_coded) {
    if (n == 0) { if (force_coded) return POR_EINVAL; if (cap < 1) return POR_ESMALL; out[0] = 0; return 1; }
    uint32_t freqs[256];
    por_histogram(plane, n, freqs);
    uint8_t lengths[256];
    uint16_t table[1 << HUF_MAX_TABLE_LOG], rev[256];
    int ok = por_ilv_lengths(freqs, lengths) && por_huf_from_lengths(lengths, table, rev);
    size_t nb = (n + ILV_BLOCK - 1) / ILV_BLOCK;
    if (ok && n <= 0xFFFFFFFFu) {
        int nw = 0;
        for (int s = 0; s < 256; s++) if (lengths[s]) nw = s + 1;
        uint8_t hdr[140];
        int64_t wl = por_huf_encode_weights(lengths, (size_t)nw, hdr, sizeof(hdr));
        size_t head = 5 + (size_t)wl;
        head += (4 - head % 4) % 4;
        size_t tab = head, data0 = tab + 4 * (nb + 1);
        /* size pass */
        size_t total = 0;
        uint32_t *words = (uint32_t *)malloc(nb * ILV_LANES * sizeof(uint32_t));
        for (size_t b = 0; b < nb; b++) {
            size_t bsz = 64;
            for (int j = 0; j < ILV_LANES; j++) {
                uint64_t bits = 0;
                for (int r = 0; r < ILV_BLOCK / (ILV_LANES * ILV_GROUP); r++) {
                    size_t g = (size_t)j + (size_t)ILV_LANES * r, a = b * ILV_BLOCK + ILV_GROUP * g;
                    for (size_t k = a; k < a + ILV_GROUP && k < n; k++) bits += lengths[plane[k]];
                }
                words[b * ILV_LANES + j] = (uint32_t)((bits + 31) / 32);
                bsz += 4 * (size_t)words[b * ILV_LANES + j];
            }
            total += bsz;
        }
        size_t best_other = ilv_all_nibbles(freqs) && ilv_packed_size(n) < 1 + n ? ilv_packed_size(n) : 1 + n;
        if ((force_coded || data0 + total < best_other) && data0 + total <= cap) {
            memset(out, 0, data0 + total);
            out[0] = 1; st32(out + 1, (uint32_t)n);
            memcpy(out + 5, hdr, (size_t)wl);
            size_t off = 0;
            for (size_t b = 0; b < nb; b++) {
                st32(out + tab + 4 * b, (uint32_t)off);
                uint8_t *blk = out + data0 + off;
                size_t wpos = 0;
                for (int j = 0; j < ILV_LANES; j++) {
                    blk[j] = (uint8_t)words[b * ILV_LANES + j];
                    uint8_t *lw = blk + 64 + 4 * wpos;
                    uint64_t acc = 0; uint32_t cnt = 0; size_t wi = 0;
                    for (int r = 0; r < ILV_BLOCK / (ILV_LANES * ILV_GROUP); r++) {
                        size_t g = (size_t)j + (size_t)ILV_LANES * r, a = b * ILV_BLOCK + ILV_GROUP * g;
                        for (size_t k = a; k < a + ILV_GROUP && k < n; k++) {
                            acc |= (uint64_t)rev[plane[k]] << cnt;
                            cnt += lengths[plane[k]];
                            if (cnt >= 32) { st32(lw + 4 * wi++, (uint32_t)acc); acc >>= 32; cnt -= 32; }
                        }
                    }
                    if (cnt) st32(lw + 4 * wi++, (uint32_t)acc);
                    wpos += words[b * ILV_LANES + j];
                }
                off += 64 + 4 * wpos;
            }
            st32(out + tab + 4 * nb, (uint32_t)off);
            free(words);
            return (int64_t)(data0 + total);
        }
        free(words);
    }
    if (force_coded) return POR_EINVAL;
    if (n <= 0xFFFFFFFFu && ilv_all_nibbles(freqs) && ilv_packed_size(n) < 1 + n) return ilv_emit_packed(plane, n, out, cap);
    if (1 + n > cap) return POR_ESMALL;
    out[0] = 0;
    memcpy(out + 1, plane, n);
    return (int64_t)(1 + n);
}

int64_t por_ilv_encode(const uint8_t *plane, size_t n, uint8_t *out, size_t cap) {
    return ilv_encode_impl(plane, n, out, cap, 0);
}

int64_t por_ilv_encode_coded(const uint8_t *plane, size_t n, uint8_t *out, size_t cap) {
    return ilv_encode_impl(plane, n, out, cap, 1);
}

int64_t por_ilv_decode(const uint8_t *p, size_t len, uint8_t *out, size_t cap) {
    if (len == 0) return POR_EINVAL;
    if (p[0] == 0) {
        if (len - 1 > cap) return POR_ESMALL;
        memcpy(out, p + 1, len - 1);
        return (int64_t)(len - 1);
    }
    if (p[0] == 2) return ilv_decode_packed(p, len, out, cap);
    if (p[0] != 1 || len < 5) return POR_EINVAL;
    size_t n = ld32(p + 1);
    if (n > cap) return POR_ESMALL;
    uint8_t w[256];
    int nw = 0;
    int64_t wl = por_huf_decode_weights(p + 5, len - 5, w, &nw);
    if (wl < 0) return POR_EINVAL;
    uint8_t lengths[256] = {0};
    for (int i = 0; i < nw; i++) { if (w[i] > HUF_MAX_TABLE_LOG) return POR_EINVAL; lengths[i] = w[i]; }
    uint16_t table[1 << HUF_MAX_TABLE_LOG];
    int mb = por_huf_from_lengths(lengths, table, NULL);
    if (!mb) return POR_EINVAL;
    size_t head = 5 + (size_t)wl;
    head += (4 - head % 4) % 4;
    size_t nb = (n + ILV_BLOCK - 1) / ILV_BLOCK, data0 = head + 4 * (nb + 1);
    if (data0 > len) return POR_EINVAL;
    size_t dlen = len - data0;
    if (ld32(p + head) != 0 || ld32(p + head + 4 * nb) != dlen) return POR_EINVAL;
    for (size_t b = 0; b < nb; b++) {
        size_t o0 = ld32(p + head + 4 * b), o1 = ld32(p + head + 4 * (b + 1));
        if (o1 < o0 || o1 > dlen || o1 - o0 < 64) return POR_EINVAL;
        const uint8_t *blk = p + data0 + o0;
        size_t wpos = 0;
        for (int j = 0; j < ILV_LANES; j++) wpos += blk[j];
        if (64 + 4 * wpos != o1 - o0) return POR_EINVAL;
        wpos = 0;
        for (int j = 0; j < ILV_LANES; j++) {
            const uint8_t *lw = blk + 64 + 4 * wpos;
            size_t nwords = blk[j], wi = 0;
            uint64_t acc = 0, used = 0; uint32_t cnt = 0;
            for (int r = 0; r < ILV_BLOCK / (ILV_LANES * ILV_GROUP); r++) {
                size_t g = (size_t)j + (size_t)ILV_LANES * r, a = b * ILV_BLOCK + ILV_GROUP * g;
                for (size_t k = a; k < a + ILV_GROUP && k < n; k++) {
                    if (cnt < 32) { if (wi < nwords) acc |= (uint64_t)ld32(lw + 4 * wi) << cnt; wi++; cnt += 32; }
                    uint16_t e = table[acc & (((uint64_t)1 << mb) - 1)];
                    out[k] = (uint8_t)e;
                    acc >>= (e >> 8); cnt -= (e >> 8); used += (e >> 8);
                }
            }
            /* a lane's words hold exactly its codes (acceptance rule) */
            if ((used + 31) / 32 != nwords) return POR_EINVAL;
            wpos += nwords;
        }
    }
    return (int64_t)n;
}

/* ------------------------------------------------------------------------- */
/* rans_ilv: this build's GPU-native interleaved rANS plane codec (no          */
/* reference counterpart; this function pair is its specification).          */
/*   [0x00][plane]  stored (empty plane: [0x00]); [0x02]... packed nibbles   */
/*   (ilv_emit_packed, as huff_ilv)                                           */
/*   [0x01][n u32][max_sym u8][f u16 x (max_sym + 1)][0-pad to 4]             */
/*        [off u32 x (nb + 1)][blocks], nb = ceil(n / 16384)                  */
/*   frequencies: the reference's normalisation (rans/compress.rs:72-135,     */
/*   11-bit, sum 2048).  Block b: [nw u32][x_j u32 x 64][w u16 x nw][0-pad    */
/*   to 4].  Step s = 0..255 (r = s / 16, t = s % 16): lanes j = 0..63 in     */
/*   order whose position P = 16384 b + 16 (64 r + j) + t is < n decode       */
/*   slot = x & 2047, x = f (x >> 11) + slot - cum, and when x < 2^16 take     */
/*   the next word: x = x << 16 | w.  The encoder starts every lane at 2^16,   */
/*   so a block is accepted iff all nw words are taken and every final        */
/*   state is 2^16.                                                            */
/* ------------------------------------------------------------------------- */

#define RILV_L (1u << 16)

static size_t rilv_pos(size_t b, int j, int s) {
    return b * ILV_BLOCK + (size_t)ILV_GROUP * ((size_t)ILV_LANES * (size_t)(s / ILV_GROUP) + (size_t)j) +
           (size_t)(s % ILV_GROUP);
}

/* force_coded: as ilv_encode_impl */
static int64_t rans_ilv_encode_impl(const uint8_t *plane, size_t n, uint8_t *out, size_t cap, int force_coded) {
    if (n == 0) { if (force_coded) return POR_EINVAL; if (cap < 1) return POR_ESMALL; out[0] = 0; return 1; }
    uint32_t raw[256];
    por_histogram(plane, n, raw);
    uint16_t f[256], cum[256];
    if (n <= 0xFFFFFFFFu && por_rans_normalize(raw, f, cum)) {
        int max_sym = 0;
        for (int i = 0; i < 256; i++) if (raw[i]) max_sym = i;
        size_t nb = (n + ILV_BLOCK - 1) / ILV_BLOCK;
        size_t head = 5 + 1 + 2 * (size_t)(max_sym + 1);
        head += (4 - head % 4) % 4;
        size_t data0 = head + 4 * (nb + 1);
        /* encode every block into scratch: words in decode order, states */
        uint16_t *words = (uint16_t *)malloc(ILV_BLOCK * sizeof(uint16_t));
        uint32_t *bw = (uint32_t *)malloc(nb * sizeof(uint32_t));
        size_t total = 0;
        for (size_t b = 0; b < nb; b++) {
            size_t nwb = 0;
            uint32_t x[ILV_LANES];
            for (int j = 0; j < ILV_LANES; j++) x[j] = RILV_L;
            for (int s = ILV_BLOCK / ILV_LANES - 1; s >= 0; s--)
                for (int j = 0; j < ILV_LANES; j++) {
                    size_t P = rilv_pos(b, j, s);
                    if (P >= n) continue;
                    uint32_t fs = f[plane[P]];
                    if ((uint64_t)x[j] >= ((uint64_t)fs << 21)) { nwb++; x[j] >>= 16; }
                    x[j] = (x[j] / fs) * 2048u + (x[j] % fs) + cum[plane[P]];
                }
            bw[b] = (uint32_t)nwb;
            total += (4 + 256 + 2 * nwb + 3) & ~(size_t)3;
        }
        size_t best_other = ilv_all_nibbles(raw) && ilv_packed_size(n) < 1 + n ? ilv_packed_size(n) : 1 + n;
        if ((force_coded || data0 + total < best_other) && data0 + total <= cap && total <= 0xFFFFFFFFu) {
            memset(out, 0, data0 + total);
            out[0] = 1; st32(out + 1, (uint32_t)n);
            out[5] = (uint8_t)max_sym;
            for (int i = 0; i <= max_sym; i++) { out[6 + 2 * i] = (uint8_t)f[i]; out[7 + 2 * i] = (uint8_t)(f[i] >> 8); }
            size_t off = 0;
            for (size_t b = 0; b < nb; b++) {
                st32(out + head + 4 * b, (uint32_t)off);
                uint8_t *blk = out + data0 + off;
                uint32_t x[ILV_LANES];
                for (int j = 0; j < ILV_LANES; j++) x[j] = RILV_L;
                size_t tail = bw[b];                     /* words fill from the end, a step at a time */
                for (int s = ILV_BLOCK / ILV_LANES - 1; s >= 0; s--) {
                    int ne = 0;
                    uint16_t ew[ILV_LANES];
                    for (int j = 0; j < ILV_LANES; j++) {
                        size_t P = rilv_pos(b, j, s);
                        if (P >= n) continue;
                        uint32_t fs = f[plane[P]];
                        if ((uint64_t)x[j] >= ((uint64_t)fs << 21)) { ew[ne++] = (uint16_t)x[j]; x[j] >>= 16; }
                        x[j] = (x[j] / fs) * 2048u + (x[j] % fs) + cum[plane[P]];
                    }
                    tail -= (size_t)ne;
                    for (int i = 0; i < ne; i++) words[tail + (size_t)i] = ew[i];
                }
                st32(blk, bw[b]);
                for (int j = 0; j < ILV_LANES; j++) st32(blk + 4 + 4 * j, x[j]);
                for (size_t i = 0; i < bw[b]; i++) { blk[260 + 2 * i] = (uint8_t)words[i]; blk[261 + 2 * i] = (uint8_t)(words[i] >> 8); }
                off += (4 + 256 + 2 * (size_t)bw[b] + 3) & ~(size_t)3;
            }
            st32(out + head + 4 * nb, (uint32_t)off);
            free(words); free(bw);
            return (int64_t)(data0 + total);
        }
        free(words); free(bw);
    }
    if (force_coded) return POR_EINVAL;
    if (n <= 0xFFFFFFFFu && ilv_all_nibbles(raw) && ilv_packed_size(n) < 1 + n) return ilv_emit_packed(plane, n, out, cap);
    if (1 + n > cap) return POR_ESMALL;
    out[0] = 0;
    memcpy(out + 1, plane, n);
    return (int64_t)(1 + n);
}

int64_t por_rans_ilv_encode(const uint8_t *plane, size_t n, uint8_t *out, size_t cap) {
    return rans_ilv_encode_impl(plane, n, out, cap, 0);
}

int64_t por_rans_ilv_encode_coded(const uint8_t *plane, size_t n, uint8_t *out, size_t cap) {
    return rans_ilv_encode_impl(plane, n, out, cap, 1);
}

int64_t por_rans_ilv_decode(const uint8_t *p, size_t len, uint8_t *out, size_t cap) {
    if (len == 0) return POR_EINVAL;
    if (p[0] == 0) {
        if (len - 1 > cap) return POR_ESMALL;
        memcpy(out, p + 1, len - 1);
        return (int64_t)(len - 1);
    }
    if (p[0] == 2) return ilv_decode_packed(p, len, out, cap);
    if (p[0] != 1 || len < 6) return POR_EINVAL;
    size_t n = ld32(p + 1);
    if (n > cap) return POR_ESMALL;
    int max_sym = p[5];
    size_t head = 5 + 1 + 2 * (size_t)(max_sym + 1);
    if (head > len) return POR_EINVAL;
    uint32_t tab[2048];
    uint32_t run = 0;
    for (int i = 0; i <= max_sym; i++) {
        uint32_t fi = (uint32_t)p[6 + 2 * i] | ((uint32_t)p[7 + 2 * i] << 8);
        if (run + fi > 2048) return POR_EINVAL;
        for (uint32_t k = 0; k < fi; k++) tab[run + k] = (uint32_t)i | (fi << 8) | (k << 20);  /* k = slot - cum */
        run += fi;
    }
    if (run != 2048) return POR_EINVAL;
    head += (4 - head % 4) % 4;
    size_t nb = (n + ILV_BLOCK - 1) / ILV_BLOCK, data0 = head + 4 * (nb + 1);
    if (data0 > len) return POR_EINVAL;
    size_t dlen = len - data0;
    for (size_t i = 5 + 1 + 2 * (size_t)(max_sym + 1); i < head; i++) if (p[i]) return POR_EINVAL;
    if (ld32(p + head) != 0 || ld32(p + head + 4 * nb) != dlen) return POR_EINVAL;
    for (size_t b = 0; b < nb; b++) {
        size_t o0 = ld32(p + head + 4 * b), o1 = ld32(p + head + 4 * (b + 1));
        if (o1 < o0 || o1 > dlen || o1 - o0 < 260) return POR_EINVAL;
        const uint8_t *blk = p + data0 + o0;
        size_t nwb = ld32(blk);
        if (((4 + 256 + 2 * nwb + 3) & ~(size_t)3) != o1 - o0) return POR_EINVAL;
        if (nwb & 1) { if (blk[260 + 2 * nwb] || blk[261 + 2 * nwb]) return POR_EINVAL; }
        uint32_t x[ILV_LANES];
        for (int j = 0; j < ILV_LANES; j++) x[j] = ld32(blk + 4 + 4 * j);
        size_t pos = 0;
        for (int s = 0; s < ILV_BLOCK / ILV_LANES; s++)
            for (int j = 0; j < ILV_LANES; j++) {
                size_t P = rilv_pos(b, j, s);
                if (P >= n) continue;
                uint32_t e = tab[x[j] & 2047u];
                out[P] = (uint8_t)e;
                x[j] = ((e >> 8) & 0xFFFu) * (x[j] >> 11) + (e >> 20);
                if (x[j] < RILV_L) {
                    if (pos >= nwb) return POR_EINVAL;
                    x[j] = (x[j] << 16) | ((uint32_t)blk[260 + 2 * pos] | ((uint32_t)blk[261 + 2 * pos] << 8));
                    pos++;
                }
            }
        if (pos != nwb) return POR_EINVAL;
        for (int j = 0; j < ILV_LANES; j++) if (x[j] != RILV_L) return POR_EINVAL;
    }
    return (int64_t)n;
}

/* ------------------------------------------------------------------------- */
/* CRC-32/ISO-HDLC (crc32fast 1.5.0), reflected poly 0xEDB88320              */
/* ------------------------------------------------------------------------- */

uint32_t por_crc32(uint32_t crc, const uint8_t *d, size_t len) {
    static uint32_t tab[256];
    static int init = 0;
    if (!init) {
        for (uint32_t i = 0; i < 256; i++) {
            uint32_t c = i;
            for (int k = 0; k < 8; k++) c = (c & 1) ? (c >> 1) ^ 0xEDB88320u : c >> 1;
            tab[i] = c;
        }
        init = 1;
    }
    crc = ~crc;
    for (size_t i = 0; i < len; i++) crc = tab[(crc ^ d[i]) & 0xFF] ^ (crc >> 8);
    return ~crc;
}

/* ------------------------------------------------------------------------- */
/* XXH64 (xxhash-rust 0.8.18 / XXH 0.8), from the published specification     */
/* ------------------------------------------------------------------------- */

#define XP1 11400714785074694791ULL
#define XP2 14029467366897019727ULL
#define XP3 1609587929392839161ULL
#define XP4 9650029242287828579ULL
#define XP5 2870177450012600261ULL
static uint64_t rotl64(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
static uint64_t xround(uint64_t acc, uint64_t in) { acc += in * XP2; acc = rotl64(acc, 31); return acc * XP1; }
static uint64_t xmerge(uint64_t acc, uint64_t v) { acc ^= xround(0, v); return acc * XP1 + XP4; }

uint64_t por_xxh64(const uint8_t *p, size_t len, uint64_t seed) {
    const uint8_t *end = p + len;
    uint64_t h;
    if (len >= 32) {
        uint64_t v1 = seed + XP1 + XP2, v2 = seed + XP2, v3 = seed, v4 = seed - XP1;
        const uint8_t *lim = end - 32;
        do {
            v1 = xround(v1, ld64(p)); v2 = xround(v2, ld64(p + 8));
            v3 = xround(v3, ld64(p + 16)); v4 = xround(v4, ld64(p + 24));
            p += 32;
        } while (p <= lim);
        h = rotl64(v1, 1) + rotl64(v2, 7) + rotl64(v3, 12) + rotl64(v4, 18);
        h = xmerge(h, v1); h = xmerge(h, v2); h = xmerge(h, v3); h = xmerge(h, v4);
    } else h = seed + XP5;
    h += (uint64_t)len;
    while (p + 8 <= end) { h ^= xround(0, ld64(p)); h = rotl64(h, 27) * XP1 + XP4; p += 8; }
    if (p + 4 <= end) { h ^= (uint64_t)ld32(p) * XP1; h = rotl64(h, 23) * XP2 + XP3; p += 4; }
    while (p < end) { h ^= (*p) * XP5; h = rotl64(h, 11) * XP1; p++; }
    h ^= h >> 33; h *= XP2; h ^= h >> 29; h *= XP3; h ^= h >> 32;
    return h;
}

/* ------------------------------------------------------------------------- */
/* BLAKE3 (hash mode), from the published specification (used for canonical  */
/* extension ids, extension/id.rs:21-30)                                      */
/* ------------------------------------------------------------------------- */

static const uint32_t B3_IV[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                                  0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};
static const int B3_PERM[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};
#define B3_CHUNK_START 1u
#define B3_CHUNK_END 2u
#define B3_PARENT 4u
#define B3_ROOT 8u
static uint32_t rotr32(uint32_t x, int r) { return (x >> r) | (x << (32 - r)); }
static void b3_g(uint32_t *s, int a, int b, int c, int d, uint32_t mx, uint32_t my) {
    s[a] = s[a] + s[b] + mx; s[d] = rotr32(s[d] ^ s[a], 16);
    s[c] = s[c] + s[d]; s[b] = rotr32(s[b] ^ s[c], 12);
    s[a] = s[a] + s[b] + my; s[d] = rotr32(s[d] ^ s[a], 8);
    s[c] = s[c] + s[d]; s[b] = rotr32(s[b] ^ s[c], 7);
}
static void b3_compress(const uint32_t cv[8], const uint32_t block[16], uint64_t counter, uint32_t blen,
                        uint32_t flags, uint32_t out[16]) {
    uint32_t s[16], m[16], t[16];
    for (int i = 0; i < 8; i++) s[i] = cv[i];
    for (int i = 0; i < 4; i++) s[8 + i] = B3_IV[i];
    s[12] = (uint32_t)counter; s[13] = (uint32_t)(counter >> 32); s[14] = blen; s[15] = flags;
    memcpy(m, block, 64);
    for (int r = 0; r < 7; r++) {
        b3_g(s, 0, 4, 8, 12, m[0], m[1]); b3_g(s, 1, 5, 9, 13, m[2], m[3]);
        b3_g(s, 2, 6, 10, 14, m[4], m[5]); b3_g(s, 3, 7, 11, 15, m[6], m[7]);
        b3_g(s, 0, 5, 10, 15, m[8], m[9]); b3_g(s, 1, 6, 11, 12, m[10], m[11]);
        b3_g(s, 2, 7, 8, 13, m[12], m[13]); b3_g(s, 3, 4, 9, 14, m[14], m[15]);
        if (r < 6) { for (int i = 0; i < 16; i++) t[i] = m[B3_PERM[i]]; memcpy(m, t, 64); }
    }
    for (int i = 0; i < 8; i++) { out[i] = s[i] ^ s[i + 8]; out[i + 8] = s[i + 8] ^ cv[i]; }
}
/* chaining value of one chunk (<= 1024 bytes); when root, returns the root output block */
static void b3_chunk(const uint32_t key[8], const uint8_t *d, size_t len, uint64_t ctr, int root, uint32_t out[16]) {
    uint32_t cv[8], blk[16], o[16];
    memcpy(cv, key, 32);
    size_t nblocks = len == 0 ? 1 : (len + 63) / 64;
    for (size_t b = 0; b < nblocks; b++) {
        uint8_t buf[64] = {0};
        size_t bl = len - b * 64 > 64 ? 64 : len - b * 64;
        if (len == 0) bl = 0;
        memcpy(buf, d + b * 64, bl);
        for (int i = 0; i < 16; i++) blk[i] = ld32(buf + 4 * i);
        uint32_t fl = (b == 0 ? B3_CHUNK_START : 0) | (b == nblocks - 1 ? B3_CHUNK_END : 0);
        if (b == nblocks - 1 && root) fl |= B3_ROOT;
        b3_compress(cv, blk, ctr, (uint32_t)bl, fl, o);
        memcpy(cv, o, 32);
        if (b == nblocks - 1) memcpy(out, o, 64);
    }
}
/* hash of a subtree of whole chunks, returning its chaining value */
static void b3_subtree(const uint8_t *d, size_t len, uint64_t ctr, int root, uint32_t out[16]) {
    if (len <= 1024) { b3_chunk(B3_IV, d, len, ctr, root, out); return; }
    /* left subtree holds the largest power-of-two number of chunks < total */
    size_t chunks = (len + 1023) / 1024, lc = 1;
    while (lc * 2 < chunks) lc *= 2;
    uint32_t l[16], r[16], blk[16];
    b3_subtree(d, lc * 1024, ctr, 0, l);
    b3_subtree(d + lc * 1024, len - lc * 1024, ctr + lc, 0, r);
    memcpy(blk, l, 32); memcpy(blk + 8, r, 32);
    b3_compress(B3_IV, blk, 0, 64, B3_PARENT | (root ? B3_ROOT : 0), out);
}
void por_blake3(const uint8_t *d, size_t len, uint8_t out[32]) {
    uint32_t o[16];
    b3_subtree(d, len, 0, 1, o);
    for (int i = 0; i < 8; i++) st32(out + 4 * i, o[i]);
}
