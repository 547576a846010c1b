/*
 * ptwm_mi355x.h -- C ABI of libptwm_mi355x.so, the MI355X (gfx950) plane
 * codec library for PTWM.
 *
 * Section 1 is the reference's native extension ABI, symbol for symbol: the
 * loader in crates/ptwm-core/src/flavor/native.rs resolves these names with
 * dlopen (native.rs:143-146, 239-311) and calls them with the signatures
 * given there.  Section 2 holds this library's own additions; the reference
 * has no counterpart for them.
 *
 * Return convention (native.rs:634-657): >= 0 is the number of bytes written
 * (never more than the stated capacity); -1 invalid input, -2 buffer too
 * small, -3 missing capability, -4 missing native dependency, -5 unsupported,
 * any other negative value an internal error.
 *
 * Device ("_cuda") entry points take device addresses as u64 and a device
 * ordinal.  They run on the library's own per-device stream (the handle the
 * *_stream_handle symbols return) and synchronise it before returning, so
 * the output is complete and visible to any stream when they return
 * (native.rs:152-162).  Input and output must be distinct allocations.
 * Calls on one device are serialised internally.
 */
#ifndef PTWM_MI355X_H
#define PTWM_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ===================================================================== */
/* 1. Reference native extension ABI                                      */
/* ===================================================================== */

/* Host-buffer plane codec, PlaneCodecFn (native.rs:62-67).  The codec is this
 * extension's own wire format ("huff_ilv", its format in ptwm_amd/csrc/huff_ilv.hip):
 * encode/decode run on device 0 through staging copies.  Encode returns -2
 * when out_len is too small. */
int64_t ptwm_plane_codec_v1_encode(const uint8_t *in, size_t in_len, uint8_t *out, size_t out_len);
int64_t ptwm_plane_codec_v1_decode(const uint8_t *in, size_t in_len, uint8_t *out, size_t out_len);

/* PlaneCodecStatefulFn (native.rs:75-83).  The codec carries no state: any
 * state_len other than 0 is rejected with -1. */
int64_t ptwm_plane_codec_v1_decode_stateful(uint8_t state_format_version, const uint8_t *state_ptr,
                                            size_t state_len, const uint8_t *in, size_t in_len,
                                            uint8_t *out, size_t out_cap);

/* PlaneCodecCudaStreamHandleFn (native.rs:150): the library's hipStream_t for
 * the device as an integer, 0 if the device is unavailable. */
uint64_t ptwm_plane_codec_v1_cuda_stream_handle(uint32_t device_ordinal);

/* PlaneCodecCudaDecodeFn (native.rs:163-174).  codec_id is a 32-byte
 * canonical id naming the payload's wire format:
 *   built-in identity / huffman / rans (ids derived for versions 1.0.0 and
 *   1.1.0, extension/builtins.rs:18-27) -> the reference plane payloads of
 *   codecs/identity.rs, codecs/huffman.rs:50-87, codecs/rans.rs:50-94;
 *   this extension's plane codec id -> its own "huff_ilv" payload.
 * Returns the decoded length; -2 if out_cap is smaller than the payload
 * declares; -1 for malformed payloads (exactly where the reference decoder
 * returns an error). */
int64_t ptwm_plane_codec_v1_decode_cuda(uint8_t state_format_version, const uint8_t *state_ptr,
                                        size_t state_len, const uint8_t *codec_id_ptr, size_t codec_id_len,
                                        uint64_t in_dev_ptr, size_t in_len, uint64_t out_dev_ptr,
                                        size_t out_cap, uint32_t device_ordinal);

/* PlaneCodecCudaEncodeFn (native.rs:185-197).  Same codec ids as decode; the
 * built-in formats are produced byte-identical to the reference encoder.
 * When out_cap is too small, writes the needed size to *needed_out and
 * returns -2. */
int64_t ptwm_plane_codec_v1_encode_cuda(uint8_t state_format_version, const uint8_t *state_ptr,
                                        size_t state_len, const uint8_t *codec_id_ptr, size_t codec_id_len,
                                        uint64_t in_dev_ptr, size_t in_len, uint64_t out_dev_ptr,
                                        size_t out_cap, uint64_t *needed_out, uint32_t device_ordinal);

/* HardwareBackendCudaStreamHandleFn (native.rs:105-111). */
uint64_t ptwm_hardware_backend_v1_cuda_stream_handle(uint32_t device_ordinal);

/* HardwareBackendCudaDispatchDecodeFn (native.rs:112-141): tensor-level
 * decode.  codec_id must be this library's decode-plan id; state_ptr holds a
 * decode plan (PTMD v1, layout in ptwm_amd/plan.py) describing one or more
 * tensors as the container stores them: chain, and per plane codec id,
 * payload offset/length inside the input buffer, decoded length, optional
 * CRC32, chunk table, inverse plane op (IntDelta, PredictorXor,
 * MantissaZeroStrip) and codec state with row layout (Order1ScaleAC).  Every tensor is restored (entropy decode + inverse
 * chain) into the output buffer at its stated offset.  Returns the number of
 * restored bytes. */
int64_t ptwm_hardware_backend_v1_dispatch_decode_cuda(uint8_t state_format_version, const uint8_t *state_ptr,
                                                      size_t state_len, const uint8_t *codec_id_ptr,
                                                      size_t codec_id_len, uint64_t in_dev_ptr, size_t in_len,
                                                      uint64_t out_dev_ptr, size_t out_len,
                                                      uint32_t device_ordinal);

/* ===================================================================== */
/* 2. Library additions (no counterpart in the reference)                 */
/* ===================================================================== */

/* Allocation-free tensor-level decode.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, plan format and results as
 * ptwm_hardware_backend_v1_dispatch_decode_cuda, for plans whose every
 * tensor takes the fused decode: planes this library's huff_ilv or rans_ilv
 * payloads (one codec per tensor, at least one coded plane, 4-byte aligned
 * in the input) or unchunked Identity planes, output 16-byte aligned, plane
 * CRC-32 only for the ieee16 / ieee32 / passthrough chains, no tensor XXH64.
 * All device scratch (descriptors, CRC tables and block partials) is one
 * fixed array of PTWM_MI355X_NOALLOC_SCRATCH_BYTES per device, and the
 * per-tensor status words a fixed 16 KiB host-coherent pinned area; both
 * are set up by ptwm_mi355x_device_init (the device's context: its stream,
 * the array's address, the status area), which the caller runs once per
 * device beforehand, and are held until the process ends.  The call itself
 * never creates the context, and calls no hipMalloc, hipFree, hipHostMalloc,
 * stream or event creation (ptwm_mi355x_alloc_calls does not move across
 * it).  Returns -3 (MissingCapability) when the device's context does not
 * exist yet or its scratch could not be resolved.  Plans outside these
 * limits (more than PTWM_MI355X_NOALLOC_MAX_TENSORS tensors, or more than
 * PTWM_MI355X_NOALLOC_MAX_CRC_BLOCKS CRC-checked 16384-byte plane blocks in
 * all) return -5 (Unsupported).  Calls on one device are serialised by the
 * library; the array keeps the last call's contents (every call rewrites
 * what it reads), so calls that overlap on one device from outside the
 * library (another process) would race. */
#define PTWM_MI355X_NOALLOC_SCRATCH_BYTES (16u << 20)
#define PTWM_MI355X_NOALLOC_MAX_TENSORS 4096u
#define PTWM_MI355X_NOALLOC_MAX_CRC_BLOCKS 883456u
int64_t ptwm_mi355x_dispatch_decode_noalloc_cuda(uint8_t state_format_version, const uint8_t *state_ptr,
                                                 size_t state_len, const uint8_t *codec_id_ptr, size_t codec_id_len,
                                                 uint64_t in_dev_ptr, size_t in_len, uint64_t out_dev_ptr,
                                                 size_t out_len, uint32_t device_ordinal);

/* Sets up the device's context (stream, pinned status words, the
 * allocation-free decode's scratch address) if it does not exist yet; every
 * other entry point does this on its first call on a device, the
 * allocation-free decode does not.  0, -1 for an invalid ordinal, -3 when
 * the allocation-free scratch could not be resolved.  No counterpart in the
 * reference: for callers that cannot allocate later. */
int64_t ptwm_mi355x_device_init(uint32_t device_ordinal);

/* Process-wide count of the library's own hipMalloc / hipHostMalloc calls
 * and stream / event creations (grow-only scratch, contexts, hashing
 * workers).  No counterpart in the reference: lets a caller check that a
 * call allocated nothing. */
uint64_t ptwm_mi355x_alloc_calls(void);

/* Cumulative counts of this device's reference-format Huffman payloads on
 * the exact route: out[0] accepted by the parallel decode, out[1] decoded
 * again by the exact state machine (malformed, or declined by the parallel
 * path's acceptance check), out[2] calls whose wavefront boundaries needed
 * more fix passes than the queued ones.  Writes min(n, 3) values, returns 3.
 * No counterpart in the reference: a caller (or a test) sees which path its
 * payloads took. */
int64_t ptwm_mi355x_decode_stats(uint32_t device_ordinal, uint64_t *out, size_t n);

/* One tensor of a container, as ptwm_mi355x_container_plan lists it (in
 * record order, the order the reference's tools list and decode them). */
typedef struct ptwm_mi355x_container_tensor {
  uint64_t name_offset;   /* the UTF-8 tensor name: byte range in the file */
  uint64_t orig_size;     /* restored bytes (the record's orig_size) */
  uint64_t out_offset;    /* where the plan restores it in the output buffer */
  uint64_t record_offset; /* the tensor record: byte range in the file */
  uint64_t record_len;
  uint32_t name_len;      /* 0 for a \x89PTWS frame (no name) */
  uint16_t dtype_code;    /* public dtype code (dtype.rs:79-103) */
  uint8_t input_format;
  uint8_t chain;          /* decode-plan chain 1..6, 0 when not planned */
  int32_t status;         /* 0 planned; -1 the record is invalid (the reference
                             fails to decode it); -5 a chain, codec or codec
                             state this library does not decode */
  int32_t plan_index;     /* its entry in the plan, -1 when not planned */
  uint32_t flags;         /* bit 0: payload XXH64 checked, bit 1: plane CRC-32s checked */
  uint32_t reserved;
} ptwm_mi355x_container_tensor;

/* Reference-side plan construction: reads a whole .ptwm file (legacy
 * \x89PTWM / \x89PTWX, compact \x89PTWC) or a \x89PTWS frame held in host
 * memory and writes the PTMD decode plan (the state bytes of
 * ptwm_hardware_backend_v1_dispatch_decode_cuda) for its tensors: payload
 * offsets index the file's own bytes, so the file copied to the device is
 * the input buffer, and the tensors are laid out at 256-byte aligned
 * offsets of an output buffer of *out_len bytes.  Replaces the open and
 * per-tensor decode set-up of container.rs:1590-1790, 1795-1892 and
 * compact.rs:407-480; the chain, codec, chunk table, plane CRC-32 and
 * payload hash of each tensor come from its record.  Writes *plan_len,
 * *n_tensors and *out_len, then the plan and the tensor list.  Returns the
 * number of planned tensors; -1 if the file's header, tables, registry or
 * index are invalid or the magic is none of these (opening it fails in the
 * reference); -2 when plan_cap or max_tensors is too small (the sizes needed
 * are written). */
int64_t ptwm_mi355x_container_plan(const uint8_t *file, size_t file_len, uint8_t *plan, size_t plan_cap,
                                   size_t *plan_len, ptwm_mi355x_container_tensor *tensors, size_t max_tensors,
                                   size_t *n_tensors, uint64_t *out_len);

/* ABI revision of this library (bumped on any incompatible change). */
/* Re-serialise a compact container (\x89PTWC, ptwc.rs) or a compact frame
 * (\x89PTWS, compact.rs) through this library's writer: the file is read
 * into its sections and records with every field kept and written again
 * (minimal varints, implicit spine edges, bound Sources, derived header,
 * index and footer), which gives a file the reference wrote back byte for
 * byte.  Returns the bytes written, -2 with *out_len set when out_cap is too
 * small, -1 for a file that does not parse, -5 for another layout.  No
 * counterpart in the reference: the writer half of container I/O
 * (ptwc.rs:77-306, tensor_record_compact.rs, compact.rs) behind the ABI. */
int64_t ptwm_mi355x_container_rewrite(const uint8_t *file, size_t file_len, uint8_t *out, size_t out_cap,
                                      size_t *out_len);

/* Write a new compact container (\x89PTWC) or, for one tensor with built-in
 * codecs and no chunks, a compact frame (\x89PTWS), from encoded planes.
 * `spec` ("PTWW" v1, layout in container_write.cpp) lists the tensors (name,
 * dtype code, input format, decode-plan chain 1..6, shape, optional XXH64)
 * and per plane its codec wire id, optional CRC-32 and chunk table, and its
 * payload's range in `payloads` (host memory).  The chains are the
 * reference's production graphs, shared through the registry with a bound
 * Source; this library's codecs (0x7F01 huff_ilv, 0x7F02 rans_ilv) go into
 * the Extension Table as third-party entries with their canonical ids
 * (tensor_record_compact.rs:137-153).  Returns the file length, -2 with
 * *out_len set when out_cap is too small, -1 for a bad spec, -5 for what the
 * layout cannot store.  No counterpart in the reference's native ABI: the
 * writer side of ptwc.rs / compact.rs for GPU-encoded planes. */
int64_t ptwm_mi355x_container_write(const uint8_t *spec, size_t spec_len, const uint8_t *payloads,
                                    size_t payloads_len, uint8_t *out, size_t out_cap, size_t *out_len);

uint32_t ptwm_mi355x_abi_version(void);

/* The canonical ids this library recognises: which = 0 own plane codec
 * (huff_ilv), 1 hardware backend, 2 decode-plan format, 3 own rANS plane
 * codec (rans_ilv).  Writes 32 bytes; returns 0 or -1. */
int64_t ptwm_mi355x_canonical_id(uint32_t which, uint8_t *out32);

/* Forward chain (bit reorder + byte/nibble split) on device: the tensor at
 * in_dev (in_len bytes) is split into planes[0..n) of plane_len bytes each.
 * chain: 1 ieee16/2-way, 2 ieee32/4-way, 3 e4m3/nibble, 4 e5m2/nibble,
 * 5 nibble split, 6 passthrough.  All addresses 16-byte aligned.  Returns the
 * plane length. */
int64_t ptwm_mi355x_split_cuda(uint32_t chain, uint64_t in_dev_ptr, size_t in_len, const uint64_t *plane_dev_ptrs,
                               uint32_t n_planes, uint32_t device_ordinal);

/* Inverse chain (merge + bit revert) on device.  Returns the tensor length. */
int64_t ptwm_mi355x_merge_cuda(uint32_t chain, const uint64_t *plane_dev_ptrs, uint32_t n_planes, size_t plane_len,
                               uint64_t out_dev_ptr, size_t out_cap, uint32_t device_ordinal);

/* Tensor-level encode (the forward counterpart of the hardware-backend decode):
 * the tensor at in_dev is split by `chain` into planes, every plane is coded
 * with this library's huff_ilv codec (stored as Identity when coding does not
 * shrink it), and the payloads are written to out_dev (256-byte aligned; each
 * payload starts at a 256-byte boundary).  A PTMD v1 decode plan describing
 * the result (payload offsets relative to out_dev) is written to plan_out and
 * its length to *plan_len_out.  Returns the bytes used in out_dev; -2 with
 * *needed_out set when out_cap is too small. */
int64_t ptwm_mi355x_encode_tensor_cuda(uint32_t chain, uint64_t in_dev_ptr, size_t in_len, uint64_t out_dev_ptr,
                                       size_t out_cap, uint8_t *plan_out, size_t plan_cap, size_t *plan_len_out,
                                       uint64_t *needed_out, uint32_t device_ordinal);

/* The same with this library's GPU-native rANS codec (rans_ilv, wire id
 * 0x7F02): every plane coded with rans_ilv, stored as Identity when coding
 * does not shrink it.  No counterpart in the reference (a new codec id). */
int64_t ptwm_mi355x_encode_tensor_rans_cuda(uint32_t chain, uint64_t in_dev_ptr, size_t in_len, uint64_t out_dev_ptr,
                                            size_t out_cap, uint8_t *plan_out, size_t plan_cap, size_t *plan_len_out,
                                            uint64_t *needed_out, uint32_t device_ordinal);

/* Tensor-level GPU encode of n_tensors tensors in one call (library
 * addition, no reference counterpart): tensor i is in_lens[i] bytes at
 * in_dev_ptrs[i] (16-byte aligned) with chain chains[i]; family 0 codes the
 * planes with huff_ilv, 1 with rans_ilv (each plane the smallest of coded,
 * packed, Identity).  Tensors are processed in batches of about 4 GiB of
 * input, each batch's planes through one histogram, size and encode pass.
 * Payloads go to out_dev_ptr (256-byte aligned) at 256-byte aligned
 * offsets; *plan_out receives one PTMD plan for all tensors, restored back
 * to back at 256-byte aligned offsets in the given order.  Returns the
 * bytes used in out; -2 with *needed_out an upper bound when out_cap is too
 * small. */
int64_t ptwm_mi355x_encode_tensors_cuda(uint32_t family, uint32_t n_tensors, const uint32_t *chains,
                                        const uint64_t *in_dev_ptrs, const uint64_t *in_lens, uint64_t out_dev_ptr,
                                        size_t out_cap, uint8_t *plan_out, size_t plan_cap, size_t *plan_len_out,
                                        uint64_t *needed_out, uint32_t device_ordinal);

/* Input bytes per batch of ptwm_mi355x_encode_tensors_cuda on the device
 * (0 = the default, 4 GiB): the size of its plane scratch.  A smaller value
 * bounds the scratch memory (more, smaller batches).  Library addition, no
 * reference counterpart.  Returns 0. */
int64_t ptwm_mi355x_set_encode_batch_bytes(uint64_t bytes, uint32_t device_ordinal);

/* Tensor-level encode into the reference's own plane formats: the tensor is
 * split by `chain`, and plane p is coded with plane_codecs[p] (wire id 0x0000
 * Identity, 0x0001 Huffman, 0x0003 rANS), in chunks of chunk_size bytes with
 * the reference's chunk frames and chunk table (compressor.rs:316-381) when
 * chunk_size > 0, else as one payload.  Every payload is byte-identical to
 * the reference encoder's (codecs/huffman.rs:37-87, codecs/rans.rs:38-94).
 * Planes start at 256-byte boundaries of out_dev (256-byte aligned; in_dev
 * 16-byte aligned).  Writes the PTMD v1 plan to plan_out (-2 with
 * *plan_len_out = needed size when plan_cap is too small); returns the bytes
 * used in out_dev, or -2 with *needed_out when out_cap is too small.
 * plane_codecs[p] = PTWM_MI355X_CODEC_SELECT picks the plane's codec by the
 * reference's trial encode (select.rs:27-64): the whole plane's Huffman,
 * rANS and Identity payload sizes, in that menu order (dispatch.rs:13-49),
 * the smallest wins and the first on ties; the plan names the winner. */
#define PTWM_MI355X_CODEC_SELECT 0xFFFFu
int64_t ptwm_mi355x_encode_tensor_ref_cuda(uint32_t chain, const uint16_t *plane_codecs, uint32_t n_codecs,
                                           uint32_t chunk_size, uint64_t in_dev_ptr, size_t in_len,
                                           uint64_t out_dev_ptr, size_t out_cap, uint8_t *plan_out, size_t plan_cap,
                                           size_t *plan_len_out, uint64_t *needed_out, uint32_t device_ordinal);

/* Tensor-level encode into the reference's plane formats with plane ops
 * (library addition): as ptwm_mi355x_encode_tensor_ref_cuda, and plane p is
 * passed through plane_ops[p] before its codec, as the reference's split
 * chains with one plane op do (python/ptwm/preprocessing/_chains.py:360-600,
 * chain/dispatch.rs:96-122): 0 none, else op | param << 8 with op
 * PTWM_MI355X_PLANE_OP_INT_DELTA (param: element width 1, 2, 4 or 8 bytes),
 * PTWM_MI355X_PLANE_OP_PREDICTOR_XOR (width 1 or 2) or
 * PTWM_MI355X_PLANE_OP_MANTISSA_ZERO_STRIP (param: k in 1..7; a plane with a
 * nonzero low k bits is refused with -1, as the reference's forward fails).
 * The plan carries the ops; the plane CRCs a caller adds cover the planes as
 * coded.  chain_trial = 1 (plane_ops ignored, may be NULL; ieee16 and ieee32
 * chains): the reference's chain trial (compressor.rs:504-640) among the
 * production variants of that chain (_chains.py:1146-1185, the plane-codec
 * ones): the plain split, IntDelta and PredictorXor on the exponent plane,
 * MantissaZeroStrip k = 1..4 on the (low) mantissa plane, in that order;
 * every variant's planes sized with plane_codecs (CODEC_SELECT: the
 * reference's selection), the smallest total of plane payloads wins, the
 * first on ties, and a variant whose op refuses its plane is skipped.
 * ops_out (may be NULL) receives the chosen op per plane.  PredictorXor is
 * one serial recurrence per plane on the device (slow on large planes). */
#define PTWM_MI355X_PLANE_OP_INT_DELTA 1u
#define PTWM_MI355X_PLANE_OP_PREDICTOR_XOR 2u
#define PTWM_MI355X_PLANE_OP_MANTISSA_ZERO_STRIP 3u
int64_t ptwm_mi355x_encode_tensor_ref_ops_cuda(uint32_t chain, const uint16_t *plane_codecs,
                                               const uint16_t *plane_ops, uint32_t n_planes, uint32_t chain_trial,
                                               uint32_t chunk_size, uint64_t in_dev_ptr, size_t in_len,
                                               uint64_t out_dev_ptr, size_t out_cap, uint8_t *plan_out,
                                               size_t plan_cap, size_t *plan_len_out, uint64_t *needed_out,
                                               uint16_t *ops_out, uint32_t device_ordinal);

/* CRC-32/ISO-HDLC of every plane of a device tensor: the tensor at in_dev is
 * split by `chain` (any alignment) and crc_out[p] receives crc32fast::hash of
 * plane p, the checksum the reference stores per plane record and verifies
 * at container.rs:2154-2159.  Returns the number of planes (n_out must be at
 * least that). */
int64_t ptwm_mi355x_plane_crc32_cuda(uint32_t chain, uint64_t in_dev_ptr, size_t in_len, uint32_t *crc_out,
                                     uint32_t n_out, uint32_t device_ordinal);

/* XXH64 with seed 0 of in_len device bytes (any alignment): the tensor
 * payload hash of container.rs:2185-2194 and compact.rs:441-445.  Serial per
 * buffer by the hash's definition, so it runs on host cores: the bytes are
 * copied to pinned host memory in chunks, after the work queued on the
 * call's stream.  Returns 0. */
int64_t ptwm_mi355x_xxh64_cuda(uint64_t in_dev_ptr, size_t in_len, uint64_t *hash_out, uint32_t device_ordinal);

/* Canonical Huffman code lengths the reference encoder assigns to a 256-bin
 * histogram (entropy/huffman/tree.rs:19-85 with the 11-bit limit of
 * :212-242), computed on the host.  Returns 0, or -1 for an all-zero
 * histogram. */
int64_t ptwm_mi355x_huffman_code_lengths(const uint32_t *freqs, uint8_t *lengths_out);

/* Stream-ordered hand-off from a producer: work already queued on
 * `producer_stream` (a hipStream_t of the device; 0 = the null stream)
 * completes before the library stream runs anything queued after this call.
 * What the reference's PyO3 layer obtains with __dlpack__(stream=<library
 * stream>) (crates/ptwm-py/src/plane_codec_cuda.rs:104-109), as one event
 * record and wait.  No counterpart in the reference C ABI.  Returns 0. */
int64_t ptwm_mi355x_stream_wait(uint64_t producer_stream, uint32_t device_ordinal);

/* use != 0: run this thread's subsequent calls for `device_ordinal` on
 * `stream` (a hipStream_t of that device, 0 = the null stream), e.g. the
 * caller's current stream, so that work queued there before a call is
 * ordered before it without an event; use == 0: the library's own stream
 * again (the default; the stream-handle entry points always return that
 * one).  Calls still complete before they return.  No counterpart in the
 * reference C ABI: the ordering the reference's PyO3 layer gets from
 * __dlpack__(stream=...) (plane_codec_cuda.rs:104-109).  Returns 0. */
int64_t ptwm_mi355x_use_stream(uint64_t stream, uint32_t use, uint32_t device_ordinal);

/* Kernel timing with HIP events recorded on the library stream around each
 * phase of the next calls on the device (off by default). */
int64_t ptwm_mi355x_set_profiling(uint32_t device_ordinal, uint32_t on);
/* Durations of the last profiled call in milliseconds: out3[0] entropy-decode
 * kernel(s), out3[1] merge kernel(s), out3[2] both. */
int64_t ptwm_mi355x_last_kernel_ms(uint32_t device_ordinal, float *out3);

#ifdef __cplusplus
}
#endif
#endif
