/*
 * ptwm_oracle.h -- CPU restatement of the PTWM plane-codec hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the correctness oracle and the
 * timed CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker.  The product
 * library (ptwm_amd/, libptwm_mi355x.so) never links, loads or calls it.
 *
 * Every function restates the reference algorithm it names (file:line under
 * the reference tree crates/ptwm-core/src/).  All arithmetic is integer.
 *
 * Return conventions: functions returning int64_t give a byte count >= 0 on
 * success and a negative POR_E* code on failure.
 */
#ifndef PTWM_ORACLE_H
#define PTWM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* error codes */
#define POR_EINVAL    (-1) /* malformed input (reference: Err(..)) */
#define POR_ESMALL    (-2) /* caller buffer too small */
#define POR_EUNSUP    (-5) /* unsupported codec / chain */

/* CompressOutcome (entropy/outcome.rs:14-50) */
#define POR_OUT_ENCODED        0
#define POR_OUT_NOT_BENEFICIAL 1
#define POR_OUT_INCOMPRESSIBLE 2
#define POR_OUT_DST_TOO_SMALL  3
#define POR_OUT_LEN_OVERFLOW   4

/* codec wire ids (codec.rs:3-23) */
#define POR_CODEC_IDENTITY 0x0000
#define POR_CODEC_HUFFMAN  0x0001
#define POR_CODEC_RANS     0x0003
#define POR_CODEC_ZSTD     0x0004
#define POR_CODEC_TANS     0x0007

/* fused chain kinds (transforms/fusion.rs) */
#define POR_CHAIN_IEEE16_SPLIT2   1 /* FusedIeee16ByteSplit2  */
#define POR_CHAIN_IEEE32_SPLIT4   2 /* FusedIeee32ByteSplit4  */
#define POR_CHAIN_E4M3_NIBBLE     3 /* FusedFp8E4M3NibbleSplit */
#define POR_CHAIN_E5M2_NIBBLE     4 /* FusedFp8E5M2NibbleSplit */
#define POR_CHAIN_NIBBLE_SPLIT    5 /* NibbleSplit (unfused, u8) */
#define POR_CHAIN_PASSTHROUGH     6 /* BytePassthrough */

/* ---- bit reorder (split/dtype8.rs, dtype16.rs, dtype32.rs) ---- */
uint8_t por_reorder_e4m3(uint8_t v);
uint8_t por_revert_e4m3(uint8_t v);
uint8_t por_reorder_e5m2(uint8_t v);
uint8_t por_revert_e5m2(uint8_t v);
uint32_t por_reorder16x2(uint32_t v);
uint32_t por_revert16x2(uint32_t v);
uint32_t por_reorder32(uint32_t v);
uint32_t por_revert32(uint32_t v);
/* whole-buffer in-place (unfused ops; trailing partial word untouched) */
void por_reorder16_buf(uint8_t *data, size_t len);
void por_revert16_buf(uint8_t *data, size_t len);
void por_reorder32_buf(uint8_t *data, size_t len);
void por_revert32_buf(uint8_t *data, size_t len);

/* ---- byte / nibble split (transforms/byte_split.rs, nibble_split.rs) ---- */
/* planes[i] must hold len/n + (i < len%n) bytes */
void por_byte_split(const uint8_t *in, size_t len, int n, uint8_t *const *planes);
/* planes all plane_len bytes; out holds plane_len*n */
void por_byte_merge(const uint8_t *const *planes, size_t plane_len, int n, uint8_t *out);
void por_nibble_split(const uint8_t *in, size_t len, uint8_t *hi, uint8_t *lo);
void por_nibble_merge(const uint8_t *hi, const uint8_t *lo, size_t len, uint8_t *out);

/* ---- fused chains (transforms/fusion.rs) ---- */
int por_chain_nplanes(int chain);
/* plane length for an input of len bytes, or -1 if len is invalid */
int64_t por_chain_plane_len(int chain, size_t len);
int por_chain_forward(int chain, const uint8_t *in, size_t len, uint8_t *const *planes);
int por_chain_inverse(int chain, const uint8_t *const *planes, size_t plane_len, uint8_t *out);

/* ---- plane ops on one terminal plane (chain/dispatch.rs:96-122); inverse
 * selects the decode direction; out may not alias in.  0 or POR_EINVAL ---- */
/* transforms/int_delta.rs: width 1, 2, 4 or 8 bytes per element */
int por_int_delta(const uint8_t *in, size_t len, unsigned width, int inverse, uint8_t *out);
/* transforms/predictor_xor.rs: fcm predictor, width 1, 2, 4 or 8 */
int por_predictor_xor(const uint8_t *in, size_t len, unsigned width, int inverse, uint8_t *out);
/* transforms/mantissa_zero.rs: k in 1..7; forward refuses nonzero low bits */
int por_mantissa_zero_strip(const uint8_t *in, size_t len, unsigned k, int inverse, uint8_t *out);

/* ---- entropy helpers ---- */
void por_histogram(const uint8_t *data, size_t len, uint32_t hist[256]);
void por_split_four(size_t len, size_t starts[4], size_t ends[4]);

/* ---- Huffman (entropy/huffman/) ---- */
/* tree.rs:19-85 + enforce_max_code_length :212-242.  Returns 1 ok, 0 None. */
int por_huf_lengths_from_freqs(const uint32_t freqs[256], uint8_t lengths[256]);
/* the same tree with the length limit max_len (1..11) instead of 11 */
int por_huf_lengths_limited(const uint32_t freqs[256], uint8_t lengths[256], int max_len);
/* tree.rs:102-177.  decode_table must hold 2048 entries.  Returns max_bits
 * or 0 if the lengths are invalid (None). rev_codes may be NULL. */
int por_huf_from_lengths(const uint8_t lengths[256], uint16_t *decode_table, uint16_t rev_codes[256]);
/* weights.rs:8-32 */
int64_t por_huf_encode_weights(const uint8_t *weights, size_t n, uint8_t *out, size_t cap);
/* weights.rs:34-85; returns bytes consumed, weights[] gets n (<=256) */
int64_t por_huf_decode_weights(const uint8_t *src, size_t len, uint8_t weights[256], int *n_out);
/* compress.rs:9-83: returns encoded length; *outcome set */
int64_t por_huf_compress(uint8_t *dst, size_t dst_cap, const uint8_t *src, size_t len, int *outcome);
/* decompress.rs:8-211 + mod.rs:34-43: exact reader state machine */
int64_t por_huf_decompress(uint8_t *dst, size_t dst_len, const uint8_t *src, size_t src_len);
/* backward bitstream writer (bitstream.rs:3-51), for tests */
int64_t por_bitwriter_pack(const uint16_t *bits, const uint8_t *nbits, size_t n, uint8_t *out, size_t cap);

/* ---- rANS (entropy/rans/) ---- */
/* compress.rs:72-122: returns 1 ok, 0 None */
int por_rans_normalize(const uint32_t raw[256], uint16_t freqs[256], uint16_t cum[256]);
int64_t por_rans_compress(uint8_t *dst, size_t dst_cap, const uint8_t *src, size_t len, int *outcome);
int64_t por_rans_decompress(uint8_t *dst, size_t dst_len, const uint8_t *src, size_t src_len);
/* EncSymbol reciprocal state update (compress.rs:35-68,164-165) */
uint32_t por_rans_enc_update(uint32_t state, uint32_t start, uint32_t freq);

/* ---- tANS (entropy/tans/mod.rs): TABLE_LOG 11, single LIFO stream ---- */
void por_tans_spread(const uint32_t norm[256], uint8_t table[2048]);
void por_tans_decode_table(const uint32_t norm[256], uint8_t sym[2048], uint8_t nb[2048], uint16_t base[2048]);
/* blob length, or 0 = store raw (incompressible / one symbol / no gain) */
int64_t por_tans_compress(uint8_t *dst, size_t cap, const uint8_t *src, size_t n);
int64_t por_tans_decompress(uint8_t *dst, size_t n, const uint8_t *src, size_t len);

/* ---- Zstd frames (codecs/zstd.rs -> zstd crate decode_all; RFC 8878), zstd_oracle.c ----
 * one or more frames into out[0..cap); decoded length, or POR_EINVAL for a
 * malformed payload or more than cap bytes */
int64_t por_zstd_decompress(uint8_t *out, size_t cap, const uint8_t *src, size_t n);

/* ---- Order1ScaleAC (codecs/order1_scale_ac.rs, range_coder.rs), o1sac_oracle.c ----
 * state: the codec state bytes ([bitmap 32 B][marginal u16 x 256][rows]);
 * row_len 0 = Flat layout (one row).  decode: n symbols or POR_EINVAL;
 * encode: payload length, POR_ESMALL if cap is too small. */
#define POR_CODEC_O1SAC 0x0011
int64_t por_o1sac_decode(const uint8_t *state, size_t state_len, unsigned state_version, const uint8_t *payload,
                         size_t payload_len, size_t row_len, uint8_t *out, size_t n);
int64_t por_o1sac_encode(const uint8_t *state, size_t state_len, const uint8_t *plane, size_t n, size_t row_len,
                         uint8_t *out, size_t cap);

/* ---- plane codec payloads (codecs/huffman.rs, codecs/rans.rs, identity.rs) ---- */
/* trial-encode selection (select.rs:27-64): every menu codec encodes the
 * plane, the smallest payload wins, the first in menu order on ties; the
 * default menu for byte planes restricted to these codecs is dispatch.rs:13-49
 * order: Huffman, Rans, (Tans, Zstd), Identity.  Returns the payload length,
 * the winner in *chosen. */
int64_t por_select_encode(const uint8_t *plane, size_t len, const uint16_t *menu, size_t menu_len,
                          uint16_t *chosen, uint8_t *out, size_t cap);
/* bound on encoded payload size for a plane of len bytes */
size_t por_codec_encode_bound(size_t len);
int64_t por_codec_encode(int codec, const uint8_t *plane, size_t len, uint8_t *out, size_t cap);
/* decode_bounded with decoded_len == max_len == cap semantics of the container
 * chunk loop: returns decoded length (may be < cap for raw tags). */
int64_t por_codec_decode(int codec, const uint8_t *payload, size_t len, uint8_t *out, size_t cap);
/* decoded length a payload declares (tag 0: raw length, tag 1: orig_len) or <0 */
int64_t por_codec_decoded_len(int codec, const uint8_t *payload, size_t len);

/* ---- chunk framing (compressor.rs:316-381, container.rs:1975-2050) ---- */
/* Encodes plane in chunk_size chunks. entries[2*k] = offset_in_payload,
 * entries[2*k+1] = decoded_size.  Returns payload length; *n_chunks set. */
int64_t por_encode_plane_chunked(int codec, const uint8_t *plane, size_t len, uint32_t chunk_size,
                                 uint8_t *out, size_t cap, uint32_t *entries, size_t max_entries,
                                 size_t *n_chunks);
int64_t por_decode_plane_chunked(int codec, const uint8_t *payload, size_t payload_len,
                                 const uint32_t *entries, size_t n_chunks, uint8_t *out, size_t cap);
/* multi-threaded (pthreads) variant used as the timed CPU baseline */
int64_t por_decode_plane_chunked_mt(int codec, const uint8_t *payload, size_t payload_len,
                                    const uint32_t *entries, size_t n_chunks, uint8_t *out,
                                    size_t cap, int threads);

/* whole-container CPU decode (tensors over threads, chunks, fused inverse):
 * the timed CPU baseline; layout of the arrays above its definition */
int64_t por_decode_tensors_mt(int codec, int chain, size_t n_tensors, const uint8_t *const *payloads,
                              const size_t *payload_lens, const uint32_t *const *entries, const size_t *n_entries,
                              uint8_t *const *outs, const size_t *out_lens, int threads);

/* per-config CPU baselines: tensors of any chain, a codec per plane, each
 * plane chunked (n_entries > 0 / chunk_sizes > 0) or one payload; chunks of
 * all planes over threads, then the inverse (forward) chain in slices.
 * Planes are tensor-major (tensor t's planes follow tensor t-1's). */
int64_t por_batch_decode_mt(size_t n_tensors, const int *chains, const size_t *out_lens, uint8_t *const *outs,
                            const int *codecs, const uint8_t *const *payloads, const size_t *payload_lens,
                            const uint32_t *const *entries, const size_t *n_entries, uint8_t *const *plane_bufs,
                            int threads);
int64_t por_batch_encode_mt(size_t n_tensors, const int *chains, const size_t *in_lens, const uint8_t *const *ins,
                            const int *codecs, const uint32_t *chunk_sizes, uint8_t *const *plane_bufs,
                            uint8_t *const *enc_outs, uint32_t *const *enc_entries, size_t *enc_lens, int threads);

/* ---- huff_ilv: this build's GPU-native plane codec (no reference
 * counterpart; its wire format is specified by these two functions).  Code
 * lengths, canonical codes and the weights header are the reference
 * Huffman's (tree.rs, weights.rs) with the length limit 6 for alphabets
 * of symbols < 16, else 11 (por_ilv_lengths); the bits are split over 64
 * lane sub-streams per 16384-symbol block. ---- */
int por_ilv_lengths(const uint32_t freqs[256], uint8_t lengths[256]);
int64_t por_ilv_encode(const uint8_t *plane, size_t len, uint8_t *out, size_t cap);
int64_t por_ilv_encode_coded(const uint8_t *plane, size_t n, uint8_t *out, size_t cap);
int64_t por_ilv_decode(const uint8_t *payload, size_t len, uint8_t *out, size_t cap);
size_t por_ilv_encode_bound(size_t len);
/* ---- rans_ilv: this build's GPU-native interleaved rANS plane codec (no
 * reference counterpart; the format is specified above por_rans_ilv_encode).
 * Encode returns the payload length (stored when coding does not shrink). */
int64_t por_rans_ilv_encode(const uint8_t *plane, size_t len, uint8_t *out, size_t cap);
int64_t por_rans_ilv_encode_coded(const uint8_t *plane, size_t n, uint8_t *out, size_t cap);
int64_t por_rans_ilv_decode(const uint8_t *payload, size_t len, uint8_t *out, size_t cap);

/* ---- integrity (crc32fast 1.5.0 / xxhash-rust 0.8.18 / blake3 1.x) ---- */
uint32_t por_crc32(uint32_t crc, const uint8_t *data, size_t len);
uint64_t por_xxh64(const uint8_t *data, size_t len, uint64_t seed);
void por_blake3(const uint8_t *data, size_t len, uint8_t out[32]);

#ifdef __cplusplus
}
#endif
#endif
