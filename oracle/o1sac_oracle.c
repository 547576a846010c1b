/*
 * o1sac_oracle.c -- CPU restatement of Order1ScaleAC (codec 0x0011).
 *
 * TEST INFRASTRUCTURE ONLY (see ptwm_oracle.h): the product library never
 * links, loads or calls it.
 *
 * Follows, under the reference tree crates/ptwm-core/src/:
 * - codecs/order1_scale_ac.rs:143-203 (state wire layout and its checks),
 *   :411-432 (row length), :449-472 (payload capacity bound), :474-486
 *   (symbol search), :593-707 (encode / decode loops);
 * - range_coder.rs:14-197 (the 32-bit carry-propagating range coder);
 * - quantize.rs:8, :50-71 (PMF total 4096, no zero entries).
 */
#include "ptwm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define O1_ALPHA 256
#define O1_TOTAL 4096u
#define O1_HDR (32 + 2 * O1_ALPHA)

typedef struct {
    uint8_t bitmap[32];
    int n_rows;
    uint32_t marginal[O1_ALPHA + 1];  /* cumulative sums */
    uint32_t (*rows)[O1_ALPHA + 1];
    uint32_t p_max;
} o1_state;

static int popcount8(uint8_t b) {
    int c = 0;
    while (b) {
        c += b & 1u;
        b >>= 1;
    }
    return c;
}

/* one PMF of 256 u16 counts -> cumulative sums; 0 if a count is zero or the
 * sum is not 4096 (validate_pmf_sum) */
static int load_pmf(const uint8_t *p, uint32_t cum[O1_ALPHA + 1], uint32_t *p_max) {
    uint32_t acc = 0;
    for (int i = 0; i < O1_ALPHA; ++i) {
        const uint32_t c = (uint32_t)p[2 * i] | ((uint32_t)p[2 * i + 1] << 8);
        if (c == 0) return 0;
        if (c > *p_max) *p_max = c;
        cum[i] = acc;
        acc += c;
    }
    cum[O1_ALPHA] = acc;
    return acc == O1_TOTAL;
}

/* deserialize_state (order1_scale_ac.rs:159-203) */
static int o1_load(const uint8_t *s, size_t len, o1_state *st) {
    memset(st, 0, sizeof(*st));
    if (len < O1_HDR) return 0;
    memcpy(st->bitmap, s, 32);
    int pop = 0;
    for (int i = 0; i < 32; ++i) pop += popcount8(st->bitmap[i]);
    if (len != (size_t)O1_HDR + (size_t)pop * 2 * O1_ALPHA) return 0;
    if (!load_pmf(s + 32, st->marginal, &st->p_max)) return 0;
    st->n_rows = pop;
    st->rows = pop ? calloc((size_t)pop, sizeof(*st->rows)) : NULL;
    if (pop && !st->rows) return 0;
    for (int r = 0; r < pop; ++r)
        if (!load_pmf(s + O1_HDR + (size_t)r * 2 * O1_ALPHA, st->rows[r], &st->p_max)) return 0;
    return 1;
}

/* cond_cumsum_for: the row of a present context (rank = present contexts
 * below it, bitmap LSB-first per byte), else the marginal */
static const uint32_t *o1_row(const o1_state *st, int prev) {
    if (prev < 0) return st->marginal;
    if (!(st->bitmap[prev >> 3] & (1u << (prev & 7)))) return st->marginal;
    int rank = 0;
    for (int i = 0; i < (prev >> 3); ++i) rank += popcount8(st->bitmap[i]);
    rank += popcount8((uint8_t)(st->bitmap[prev >> 3] & ((1u << (prev & 7)) - 1u)));
    return st->rows[rank];
}

/* max_decodable_len (order1_scale_ac.rs:449-472) */
static uint64_t o1_capacity(const o1_state *st, size_t payload_len) {
    if (st->p_max == 0 || st->p_max >= O1_TOTAL) return UINT64_MAX;
    const double bits = log2((double)O1_TOTAL / (double)st->p_max);
    const double budget = 8.0 * (double)(payload_len > 5 ? payload_len - 5 : 0);
    const double n = floor(budget / bits) + 1.0;
    return n >= 18446744073709551615.0 ? UINT64_MAX : (uint64_t)n;
}

int64_t por_o1sac_decode(const uint8_t *state, size_t state_len, unsigned state_version, const uint8_t *payload,
                         size_t payload_len, size_t row_len, uint8_t *out, size_t n) {
    if (state_version != 1) return POR_EINVAL;
    o1_state st;
    if (!o1_load(state, state_len, &st)) {
        free(st.rows);
        return POR_EINVAL;
    }
    const size_t rl = row_len ? row_len : (n ? n : 1);  /* Flat: the whole plane is one row */
    if (n % rl || (uint64_t)n > o1_capacity(&st, payload_len)) {
        free(st.rows);
        return POR_EINVAL;
    }
    /* RangeDecoder::new: five bytes preloaded (the first is the encoder's
     * alignment byte); bytes past the payload read as zero */
    uint64_t low = 0, range = 0xFFFFFFFFu, code = 0;
    size_t pos = 0;
    for (; pos < 5; ++pos) code = (code << 8) | (pos < payload_len ? payload[pos] : 0u);
    int prev = -1;
    size_t row_pos = 0;
    for (size_t i = 0; i < n; ++i) {
        if (row_pos == 0) prev = -1;
        const uint32_t *cum = o1_row(&st, prev);
        const uint64_t rpt = range / O1_TOTAL;
        const uint64_t offset = ((code & 0xFFFFFFFFu) - low) & 0xFFFFFFFFu;
        uint64_t target = offset / rpt;
        if (target > O1_TOTAL - 1) target = O1_TOTAL - 1;
        size_t lo = 0, hi = O1_ALPHA;  /* binary_search_cumsum */
        while (lo + 1 < hi) {
            const size_t mid = (lo + hi) / 2;
            if (cum[mid] <= target) lo = mid;
            else hi = mid;
        }
        const uint32_t c0 = cum[lo], p = cum[lo + 1] - c0;
        low += (uint64_t)c0 * rpt;  /* RangeDecoder::advance */
        range = (uint64_t)p * rpt;
        low &= 0xFFFFFFFFu;
        while (range < (1u << 24)) {
            const uint64_t b = pos < payload_len ? payload[pos] : 0u;
            ++pos;
            code = ((code & 0xFFFFFFFFFFull) << 8) | b;
            low = (low & 0xFFFFFFu) << 8;
            range <<= 8;
        }
        out[i] = (uint8_t)lo;
        prev = (int)lo;
        row_pos = (row_pos + 1) % rl;
    }
    free(st.rows);
    return (int64_t)n;
}

/* RangeEncoder (range_coder.rs:15-120) */
typedef struct {
    uint64_t low, range;
    uint8_t cache;
    uint32_t cache_size;
    uint8_t *out;
    size_t len, cap;
    int overflow;
} o1_enc;

static void enc_put(o1_enc *e, uint8_t b) {
    if (e->len < e->cap) e->out[e->len] = b;
    else e->overflow = 1;
    e->len++;
}

static void enc_shift_low(o1_enc *e) {
    const uint8_t carry = (uint8_t)(e->low >> 32);
    const uint8_t top = (uint8_t)((e->low >> 24) & 0xFFu);
    if (top == 0xFF && carry == 0) {
        e->cache_size++;
    } else {
        enc_put(e, (uint8_t)(e->cache + carry));
        for (uint32_t k = 0; k < e->cache_size; ++k) enc_put(e, carry ? 0x00 : 0xFF);
        e->cache_size = 0;
        e->cache = top;
    }
    e->low = (e->low & 0xFFFFFFu) << 8;
}

int64_t por_o1sac_encode(const uint8_t *state, size_t state_len, const uint8_t *plane, size_t n, size_t row_len,
                         uint8_t *out, size_t cap) {
    o1_state st;
    if (!o1_load(state, state_len, &st)) {
        free(st.rows);
        return POR_EINVAL;
    }
    const size_t rl = row_len ? row_len : (n ? n : 1);
    if (n % rl) {
        free(st.rows);
        return POR_EINVAL;
    }
    o1_enc e = {0, 0xFFFFFFFFu, 0, 0, out, 0, cap, 0};
    for (size_t i = 0; i < n; ++i) {
        const int prev = i % rl == 0 ? -1 : plane[i - 1];
        const uint32_t *cum = o1_row(&st, prev);
        const uint32_t c0 = cum[plane[i]], p = cum[plane[i] + 1] - c0;
        const uint64_t rpt = e.range / O1_TOTAL;
        e.low += (uint64_t)c0 * rpt;
        e.range = (uint64_t)p * rpt;
        while (e.range < (1u << 24)) {
            enc_shift_low(&e);
            e.range <<= 8;
        }
    }
    for (int k = 0; k < 5; ++k) enc_shift_low(&e);
    enc_put(&e, e.cache);
    for (uint32_t k = 0; k < e.cache_size; ++k) enc_put(&e, 0xFF);
    free(st.rows);
    if (e.overflow) return POR_ESMALL;
    return (int64_t)e.len;
}
