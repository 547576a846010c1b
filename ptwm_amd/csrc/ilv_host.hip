// ilv_host.hip -- host orchestration of the huff_ilv encoder and decoder.
//
// Encode (per call, any number of planes): histogram kernel -> host code
// tables (huffman_host.cpp) -> size kernel -> host prefix sums and payload
// layout -> encode kernel plus header / offset-table uploads.  Each plane
// takes the smallest payload form (ilv_choose_form): coded, packed nibbles
// or stored.
//
// Decode: tensors are grouped by chain and decoded with one fused launch per
// chain (ilv_decode_kernel<chain>): persistent workgroups (as many as fit on
// the device at the launch's LDS size) over 4-block tiles.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

#include "huff_ilv.h"
#include "huffman_host.h"
#include "ilv_host.h"
#include "integrity.h"
#include "rans_ilv.h"
#include "runtime.h"

namespace ptwm {

static inline uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

uint32_t ilv_choose_form(uint64_t n, bool nibbles, bool codable, uint64_t coded_len, bool identity_fallback,
                         uint64_t* len) {
  const uint64_t stored = n + 1, packed = kPackedHeadBytes + (n + 1) / 2;
  const bool pack_ok = nibbles && packed < stored;
  const uint64_t other = pack_ok ? packed : stored;
  uint32_t form = kFormStored;
  uint64_t l = stored;
  if (codable && coded_len < other) {
    form = kFormCoded;
    l = coded_len;
  } else if (pack_ok) {
    form = kFormPacked;
    l = packed;
  }
  if (identity_fallback && (form == kFormStored || l >= n)) {
    form = kFormIdentity;
    l = n;
  }
  *len = l;
  return form;
}

int64_t ilv_store_planes(DevCtx& ctx, const uint64_t* src, const uint64_t* n, uint32_t np, uint64_t out_dev,
                         const IlvEncResult* res, const uint32_t* form, std::vector<uint8_t>& keep) {
  hipStream_t s = ctx.stream;
  // [8 header bytes per plane][pack jobs][store jobs]; the job arrays go
  // to the device in one upload
  keep.assign((size_t)np * (8 + sizeof(IlvPackJob) + sizeof(IlvStoreJob)), 0);
  IlvPackJob* jobs = reinterpret_cast<IlvPackJob*>(keep.data() + 8 * np);
  IlvStoreJob* sjobs = reinterpret_cast<IlvStoreJob*>(keep.data() + (8 + sizeof(IlvPackJob)) * (size_t)np);
  uint32_t nj = 0, ns = 0;
  uint64_t max_n = 0, max_s = 0;
  for (uint32_t p = 0; p < np; ++p) {
    const uint64_t dst = out_dev + res[p].offset;
    uint8_t* head = keep.data() + 8 * p;
    if (form[p] == kFormIdentity || form[p] == kFormStored) {
      const uint32_t shift = form[p] == kFormStored ? 1u : 0u;
      if (n[p] + shift == 0) continue;
      sjobs[ns++] = IlvStoreJob{src[p], dst, n[p], shift, 0};
      max_s = std::max(max_s, n[p] + shift);
    } else if (form[p] == kFormPacked) {
      head[0] = 2;
      const uint32_t nn = (uint32_t)n[p];
      std::memcpy(head + 1, &nn, 4);
      PTWM_HIP_TRY(hipMemcpyAsync(reinterpret_cast<void*>(dst), head, kPackedHeadBytes, hipMemcpyHostToDevice, s));
      jobs[nj++] = IlvPackJob{src[p], dst + kPackedHeadBytes, n[p]};
      max_n = std::max(max_n, n[p]);
    }
  }
  if (nj || ns) {
    const size_t pack_bytes = nj * sizeof(IlvPackJob);
    PTWM_HIP_TRY(ctx.enc_pack.ensure(pack_bytes + ns * sizeof(IlvStoreJob)));
    if (ns) std::memmove(reinterpret_cast<uint8_t*>(jobs) + pack_bytes, sjobs, ns * sizeof(IlvStoreJob));
    PTWM_HIP_TRY(hipMemcpyAsync(ctx.enc_pack.ptr, jobs, pack_bytes + ns * sizeof(IlvStoreJob), hipMemcpyHostToDevice,
                                s));
    uint8_t* d = static_cast<uint8_t*>(ctx.enc_pack.ptr);
    PTWM_HIP_TRY(launch_ilv_pack(reinterpret_cast<const IlvPackJob*>(d), nj, max_n, s));
    PTWM_HIP_TRY(launch_ilv_store(reinterpret_cast<const IlvStoreJob*>(d + pack_bytes), ns, max_s, s));
  }
  return kOk;
}

int64_t ilv_encode_planes(DevCtx& ctx, const uint64_t* src, const uint64_t* n, uint32_t np, uint64_t out_dev,
                          uint64_t out_cap, bool identity_fallback, IlvEncResult* res, uint64_t* needed) {
  hipStream_t s = ctx.stream;
  if (np == 0) return 0;
  for (uint32_t p = 0; p < np; ++p)
    if ((src[p] & 15u) != 0 || n[p] > 0xFFFFFFFFull) return kInvalidInput;
  // ---- histograms ----
  std::vector<IlvEncPlane> hp(np);
  uint64_t max_n = 0;
  for (uint32_t p = 0; p < np; ++p) {
    hp[p] = IlvEncPlane{src[p], n[p], p, 0};
    max_n = std::max(max_n, n[p]);
  }
  PTWM_HIP_TRY(ctx.enc_planes.ensure(np * sizeof(IlvEncPlane)));
  PTWM_HIP_TRY(ctx.enc_hist.ensure(np * 256 * sizeof(uint32_t)));
  PTWM_HIP_TRY(ctx.h_enc.ensure(np * 256 * sizeof(uint32_t) + np * sizeof(IlvEncPlane)));
  std::memcpy(ctx.h_enc.ptr, hp.data(), np * sizeof(IlvEncPlane));
  PTWM_HIP_TRY(hipMemcpyAsync(ctx.enc_planes.ptr, ctx.h_enc.ptr, np * sizeof(IlvEncPlane), hipMemcpyHostToDevice, s));
  PTWM_HIP_TRY(hipMemsetAsync(ctx.enc_hist.ptr, 0, np * 256 * sizeof(uint32_t), s));
  PTWM_HIP_TRY(launch_ilv_hist(static_cast<const IlvEncPlane*>(ctx.enc_planes.ptr), np, max_n,
                               static_cast<uint32_t*>(ctx.enc_hist.ptr), s));
  std::vector<uint32_t> hist(np * 256);
  PTWM_HIP_TRY(hipMemcpyAsync(hist.data(), ctx.enc_hist.ptr, np * 256 * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
  PTWM_HIP_TRY(hipStreamSynchronize(s));
  // ---- code tables ----
  std::vector<uint32_t> codes(np * 256, 0);
  std::vector<std::vector<uint8_t>> weights(np);
  std::vector<uint8_t> codable(np, 0);
  // planes are independent (each writes its own entries): spread large
  // batches over host threads
  auto build_codes = [&](uint32_t p0, uint32_t p1) {
    for (uint32_t p = p0; p < p1; ++p) {
      if (n[p] == 0) continue;
      uint8_t lengths[256];
      uint16_t rev[256];
      if (!ilv_lengths_from_freqs(&hist[256 * p], lengths)) continue;
      if (!huf_canonical(lengths, rev)) continue;
      for (int sy = 0; sy < 256; ++sy) codes[256 * p + sy] = ((uint32_t)lengths[sy] << 16) | rev[sy];
      uint8_t w[140];
      int wl = huf_encode_weights(lengths, w);
      if (wl < 0) continue;
      // a coded payload is at least its header, offset table, lane counts
      // and ceil(code bits / 8): a plane for which that is not shorter than
      // the stored or packed form is not sized (the form choice below would
      // not take the coded form)
      uint64_t bits = 0;
      for (int sy = 0; sy < 256; ++sy) bits += (uint64_t)hist[256 * p + sy] * lengths[sy];
      const uint64_t nb = (n[p] + kIlvBlock - 1) / kIlvBlock;
      const uint64_t lower = align_up(5 + (uint64_t)wl, 4) + 4 * (nb + 1) + 64 * nb + (bits + 7) / 8;
      const uint64_t stored = n[p] + 1, packed = kPackedHeadBytes + (n[p] + 1) / 2;
      const uint64_t other = all_nibbles(&hist[256 * p]) && packed < stored ? packed : stored;
      if (lower >= other) continue;
      weights[p].assign(w, w + wl);
      codable[p] = 1;
    }
  };
  const uint32_t hw = std::max(1u, std::thread::hardware_concurrency());
  const uint32_t nthr = np >= 64 ? std::min<uint32_t>(std::min<uint32_t>(hw, 8), np / 16) : 1;
  if (nthr <= 1) {
    build_codes(0, np);
  } else {
    std::vector<std::thread> pool;
    for (uint32_t t = 0; t < nthr; ++t)
      pool.emplace_back(build_codes, (uint32_t)((uint64_t)np * t / nthr), (uint32_t)((uint64_t)np * (t + 1) / nthr));
    for (std::thread& th : pool) th.join();
  }
  // ---- size pass over every block of every codable plane ----
  std::vector<IlvEncBlock> blocks;
  std::vector<uint32_t> first_block(np, 0), nbs(np, 0);
  for (uint32_t p = 0; p < np; ++p) {
    first_block[p] = (uint32_t)blocks.size();
    if (!codable[p]) continue;
    nbs[p] = (uint32_t)((n[p] + kIlvBlock - 1) / kIlvBlock);
    for (uint32_t b = 0; b < nbs[p]; ++b) blocks.push_back(IlvEncBlock{0, p, b, 0, 0});
  }
  const uint32_t nblk = (uint32_t)blocks.size();
  std::vector<uint32_t> bbytes(nblk);
  if (nblk) {
    PTWM_HIP_TRY(ctx.enc_codes.ensure(codes.size() * sizeof(uint32_t)));
    PTWM_HIP_TRY(ctx.enc_blocks.ensure(nblk * sizeof(IlvEncBlock)));
    PTWM_HIP_TRY(ctx.enc_lane_words.ensure((size_t)nblk * 64));
    PTWM_HIP_TRY(ctx.enc_block_bytes.ensure(nblk * sizeof(uint32_t)));
    PTWM_HIP_TRY(ctx.h_enc.ensure(codes.size() * 4 + nblk * sizeof(IlvEncBlock) + nblk * 4 + 64));
    uint8_t* hb = static_cast<uint8_t*>(ctx.h_enc.ptr);
    std::memcpy(hb, codes.data(), codes.size() * 4);
    std::memcpy(hb + codes.size() * 4, blocks.data(), nblk * sizeof(IlvEncBlock));
    PTWM_HIP_TRY(hipMemcpyAsync(ctx.enc_codes.ptr, hb, codes.size() * 4, hipMemcpyHostToDevice, s));
    PTWM_HIP_TRY(hipMemcpyAsync(ctx.enc_blocks.ptr, hb + codes.size() * 4, nblk * sizeof(IlvEncBlock),
                                hipMemcpyHostToDevice, s));
    PTWM_HIP_TRY(launch_ilv_size(static_cast<const IlvEncPlane*>(ctx.enc_planes.ptr),
                                 static_cast<const IlvEncBlock*>(ctx.enc_blocks.ptr), nblk,
                                 static_cast<const uint32_t*>(ctx.enc_codes.ptr),
                                 static_cast<uint8_t*>(ctx.enc_lane_words.ptr),
                                 static_cast<uint32_t*>(ctx.enc_block_bytes.ptr), s));
    PTWM_HIP_TRY(hipMemcpyAsync(bbytes.data(), ctx.enc_block_bytes.ptr, nblk * 4, hipMemcpyDeviceToHost, s));
    PTWM_HIP_TRY(hipStreamSynchronize(s));
  }
  // ---- layout: payloads at 256-byte aligned offsets ----
  uint64_t off = 0;
  std::vector<uint64_t> head(np, 0);
  std::vector<uint32_t> form(np, kFormStored);
  for (uint32_t p = 0; p < np; ++p) {
    off = align_up(off, 256);
    res[p].offset = off;
    uint64_t pay = 0;
    bool codable_p = codable[p];
    if (codable_p) {
      uint64_t d = 0;
      for (uint32_t b = 0; b < nbs[p]; ++b) d += bbytes[first_block[p] + b];
      head[p] = align_up(5 + weights[p].size(), 4);
      pay = head[p] + 4ull * (nbs[p] + 1) + d;
      codable_p = d <= 0xFFFFFFFFull;
    }
    form[p] = ilv_choose_form(n[p], all_nibbles(&hist[256 * p]), codable_p, pay, identity_fallback, &res[p].len);
    res[p].coded = form[p] == kFormCoded ? 1 : 0;
    res[p].codec = form[p] == kFormIdentity ? kCodecIdentity : kCodecHuffIlv;
    off += res[p].len;
  }
  const uint64_t total = off;
  if (total > out_cap) {
    if (needed) *needed = total;
    return kBufferTooSmall;
  }
  // ---- headers, offset tables and block destinations ----
  uint64_t host_bytes = 0;
  for (uint32_t p = 0; p < np; ++p)
    if (res[p].coded) host_bytes += head[p] + 4ull * (nbs[p] + 1);
  PTWM_HIP_TRY(ctx.h_enc.ensure(host_bytes + nblk * sizeof(IlvEncBlock) + 64));
  uint8_t* hb = static_cast<uint8_t*>(ctx.h_enc.ptr);
  IlvEncBlock* hblk = reinterpret_cast<IlvEncBlock*>(hb + host_bytes);
  std::memcpy(hblk, blocks.data(), nblk * sizeof(IlvEncBlock));
  std::vector<uint8_t> keep;
  if (int64_t rc = ilv_store_planes(ctx, src, n, np, out_dev, res, form.data(), keep); rc != kOk) return rc;
  uint64_t hoff = 0;
  for (uint32_t p = 0; p < np; ++p) {
    const uint64_t dst = out_dev + res[p].offset;
    if (!res[p].coded) continue;
    uint8_t* h = hb + hoff;
    std::memset(h, 0, head[p]);
    h[0] = 1;
    uint32_t nn = (uint32_t)n[p];
    std::memcpy(h + 1, &nn, 4);
    std::memcpy(h + 5, weights[p].data(), weights[p].size());
    uint32_t* tab = reinterpret_cast<uint32_t*>(h + head[p]);
    uint64_t acc = 0;
    const uint64_t data_dev = dst + head[p] + 4ull * (nbs[p] + 1);
    for (uint32_t b = 0; b < nbs[p]; ++b) {
      tab[b] = (uint32_t)acc;
      hblk[first_block[p] + b].dst = data_dev + acc;
      acc += bbytes[first_block[p] + b];
    }
    tab[nbs[p]] = (uint32_t)acc;
    const uint64_t hl = head[p] + 4ull * (nbs[p] + 1);
    PTWM_HIP_TRY(hipMemcpyAsync(reinterpret_cast<void*>(dst), h, hl, hipMemcpyHostToDevice, s));
    hoff += hl;
  }
  if (nblk) {
    // only blocks of coded planes are written; lw keeps the size-pass index
    uint32_t live = 0, max_words = 0;
    for (uint32_t i = 0; i < nblk; ++i)
      if (res[hblk[i].plane].coded) {
        IlvEncBlock bk = hblk[i];
        bk.lw = i;
        hblk[live++] = bk;
        max_words = std::max(max_words, bbytes[i] >= 64 ? (bbytes[i] - 64) / 4 : 0u);
      }
    // LDS for the largest block's words, within the cap (larger blocks are
    // written lane by lane)
    const uint32_t stage_words = std::min<uint32_t>(kIlvEncStageMax, (max_words + 3) & ~3u);
    if (live) {
      PTWM_HIP_TRY(hipMemcpyAsync(ctx.enc_blocks.ptr, hblk, live * sizeof(IlvEncBlock), hipMemcpyHostToDevice, s));
      PTWM_HIP_TRY(launch_ilv_encode(static_cast<const IlvEncPlane*>(ctx.enc_planes.ptr),
                                     static_cast<const IlvEncBlock*>(ctx.enc_blocks.ptr), live,
                                     static_cast<const uint32_t*>(ctx.enc_codes.ptr),
                                     static_cast<const uint8_t*>(ctx.enc_lane_words.ptr), stage_words, s));
    }
  }
  PTWM_HIP_TRY(hipStreamSynchronize(s));
  return (int64_t)total;
}

int64_t ilv_decode_tensors(DevCtx& ctx, const std::vector<IlvTensor>& tensors_in, bool all_slots) {
  hipStream_t s = ctx.stream;
  if (tensors_in.empty()) return kOk;
  std::vector<IlvTensor> tensors = tensors_in;
  const size_t nt = tensors.size();
  if (ctx.cu_count <= 0) {
    PTWM_HIP_TRY(hipDeviceGetAttribute(&ctx.cu_count, hipDeviceAttributeMultiprocessorCount, ctx.dev));
    if (ctx.cu_count <= 0) ctx.cu_count = 1;
  }
  // Coded payloads are read as 32-bit words: copy the ones that do not
  // start on a 4-byte boundary to aligned scratch first.
  uint64_t realign_bytes = 0;
  for (const IlvTensor& T : tensors)
    for (uint32_t p = 0; p < T.n_planes; ++p)
      if (T.planes[p].coded && (T.planes[p].base & 3u)) realign_bytes = align_up(realign_bytes + T.planes[p].len, 256);
  if (realign_bytes) {
    // one batched copy for all of them (chunk frames put most payloads of a
    // chunked plane off 4-byte boundaries)
    PTWM_HIP_TRY(ctx.ilv_realign.ensure(realign_bytes));
    std::vector<IlvStoreJob> jobs;
    uint64_t off = 0, max_n = 0;
    for (IlvTensor& T : tensors)
      for (uint32_t p = 0; p < T.n_planes; ++p) {
        IlvPlane& P = T.planes[p];
        if (!P.coded || !(P.base & 3u)) continue;
        const uint64_t dst = reinterpret_cast<uint64_t>(ctx.ilv_realign.ptr) + off;
        jobs.push_back(IlvStoreJob{P.base, dst, P.len, 0, 0});
        max_n = P.len > max_n ? P.len : max_n;
        P.base = dst;
        off = align_up(off + P.len, 256);
      }
    const size_t jb = jobs.size() * sizeof(IlvStoreJob);
    PTWM_HIP_TRY(ctx.realign_jobs.ensure(jb));
    PTWM_HIP_TRY(ctx.h_realign.ensure(jb));
    std::memcpy(ctx.h_realign.ptr, jobs.data(), jb);
    PTWM_HIP_TRY(hipMemcpyAsync(ctx.realign_jobs.ptr, ctx.h_realign.ptr, jb, hipMemcpyHostToDevice, s));
    PTWM_HIP_TRY(launch_ilv_realign(static_cast<const IlvStoreJob*>(ctx.realign_jobs.ptr), (uint32_t)jobs.size(),
                                    max_n, s));
  }
  // One persistent launch per chain present.  Per launch: the tensor list,
  // its 4-block tile prefix sums, the LDS table slots (most coded planes of
  // any tensor) and the staging words per wavefront: the largest estimated
  // block of any tensor (coded payload words per block, +2%, rounded up),
  // capped by the workgroup LDS budget.  Blocks above it take the kernel's
  // global-memory path.
  struct Launch {
    uint32_t family, chain, first, m, slots, stage_words, grid;
    bool crc;  // some tensor of the launch has fused CRC partials (huff_ilv family)
  };
  std::vector<Launch> launches;
  // The launch chain codes of a family: one per chain present, except that
  // huff_ilv nibble-split and passthrough tensors (MXFP4 weights and their
  // scales) share one two-chain launch when none of them has fused CRC
  // partials (the two-chain kernel has no CRC variant).
  bool pair_ok = false;
  {
    bool has5 = false, has6 = false, crc56 = false;
    for (const IlvTensor& T : tensors) {
      if (T.family != kFamilyHuff || T.n == 0) continue;
      has5 |= T.chain == kChainNibbleSplit;
      has6 |= T.chain == kChainPassthrough;
      crc56 |= (T.chain == kChainNibbleSplit || T.chain == kChainPassthrough) && T.crc_first != kIlvNoCrc;
    }
    pair_ok = has5 && has6 && !crc56;
  }
  auto launch_codes = [&](uint32_t fam) {
    std::vector<uint32_t> codes{kChainIeee16Split2, kChainIeee32Split4, kChainE4m3Nibble, kChainE5m2Nibble};
    if (fam == kFamilyHuff && pair_ok) {
      codes.push_back(kIlvPairNibblePass);
    } else {
      codes.push_back(kChainNibbleSplit);
      codes.push_back(kChainPassthrough);
    }
    return codes;
  };
  std::vector<uint32_t> idx;  // per launch: [m + 1 prefix][m tensor indexes]
  // Within a launch, the tensors whose tiles build decode tables come first:
  // the workgroups of the last tiles start a few microseconds late and set
  // up under the others' streaming traffic, so the tiles with the longest
  // setup (table builds and staging) go to the first workgroups (MXFP4: the
  // coded E8M0 scales ahead of the packed weights).
  std::vector<uint32_t> order;
  order.reserve(nt);
  for (int pass = 0; pass < 2; ++pass)
    for (uint32_t ti = 0; ti < nt; ++ti) {
      const IlvTensor& T = tensors[ti];
      bool tables = false;
      for (uint32_t p = 0; p < T.n_planes; ++p) {
        const IlvPlane& P = T.planes[p];
        tables |= P.coded && P.len != T.n + 1 && P.len != kPackedHeadBytes + (T.n + 1) / 2;
      }
      if (tables == (pass == 0)) order.push_back(ti);
    }
  for (uint32_t fam = kFamilyHuff; fam <= kFamilyRans; ++fam)
  for (uint32_t chain : launch_codes(fam)) {
    std::vector<uint32_t> tix, tpre{0};
    uint32_t slots = 0;
    uint64_t est = 0;
    bool crc = false;
    for (const uint32_t ti : order) {
      const IlvTensor& T = tensors[ti];
      if (T.family != fam || !ilv_code_has(chain, T.chain) || T.n == 0) continue;
      if (T.crc_first != kIlvNoCrc) {
        if (fam != kFamilyHuff) return kInternal;
        crc = true;
      }
      const uint64_t nb = (T.n + kIlvBlock - 1) / kIlvBlock;
      // LDS table slots and staging for the planes that may be coded: a
      // native payload of the stored (n + 1) or packed (8 + ceil(n / 2))
      // length is taken as such.  A coded plane of either length finds no
      // slot, and its tensor is decoded again with a slot for every plane
      // (kIlvRetrySlots); its blocks may take the kernel's global-memory path.
      uint32_t need_slots = 0;
      uint64_t words = fam == kFamilyHuff ? 4 : 0;
      for (uint32_t p = 0; p < T.n_planes; ++p) {
        const IlvPlane& P = T.planes[p];
        if (!P.coded) continue;
        if (!all_slots && (P.len == T.n + 1 || P.len == kPackedHeadBytes + (T.n + 1) / 2)) continue;
        ++need_slots;
        const uint64_t per_block = (T.planes[p].len + 4 * nb - 1) / (4 * nb);
        // huff_ilv nibble chains may carry fixed-length codes: room for the
        // kernel's per-lane skew of equal-length lane streams (two words per lane)
        const uint64_t skew =
            fam == kFamilyRans || T.chain == kChainIeee16Split2 || T.chain == kChainIeee32Split4 ? 0 : 128;
        words += align_up(per_block + per_block / 50 + skew + 4, 4);
      }
      slots = std::max(slots, need_slots);
      est = std::max(est, words);
      tix.push_back(ti);
      tpre.push_back(tpre.back() + (uint32_t)((nb + kIlvBlocksPerTile - 1) / kIlvBlocksPerTile));
    }
    if (tix.empty()) continue;
    const uint64_t max_lds = fam == kFamilyHuff ? kIlvMaxLds : kRilvMaxLds;
    const uint64_t fixed =
        fam == kFamilyHuff ? ilv_decode_lds_bytes(chain, slots, 0, crc) : rilv_decode_lds_bytes(chain, slots, 0);
    uint64_t cap_words = ((max_lds - std::min<uint64_t>(fixed, max_lds)) / 16) & ~3ull;
    // the staging area also holds the payload heads at a tensor's start
    const uint64_t head_min = fam == kFamilyHuff ? kIlvHeadWords : kRilvHeadWords;  // 4 planes over 4 wavefronts
    uint64_t stage = align_up(std::max<uint64_t>(std::max<uint64_t>(est, 8), head_min), 4);
    if (stage > cap_words) stage = cap_words;
    if (stage < head_min) return kInternal;
    int per_cu = 0;
    const uint64_t occ_key =
        (uint64_t)chain | ((uint64_t)slots << 12) | (stage << 20) | ((uint64_t)crc << 61) | ((uint64_t)fam << 62);
    auto it = ctx.ilv_occupancy.find(occ_key);
    if (it != ctx.ilv_occupancy.end()) {
      per_cu = it->second;
    } else {
      if (fam == kFamilyHuff) PTWM_HIP_TRY(ilv_decode_occupancy(chain, slots, (uint32_t)stage, crc, &per_cu));
      else PTWM_HIP_TRY(rilv_decode_occupancy(chain, slots, (uint32_t)stage, &per_cu));
      ctx.ilv_occupancy[occ_key] = per_cu;
    }
    if (per_cu < 1) per_cu = 1;
    const uint64_t n_tiles = tpre.back();
    const uint32_t grid = (uint32_t)std::min<uint64_t>(n_tiles, (uint64_t)per_cu * ctx.cu_count);
    launches.push_back(Launch{fam, chain, (uint32_t)idx.size(), (uint32_t)tix.size(), slots, (uint32_t)stage, grid, crc});
    idx.insert(idx.end(), tpre.begin(), tpre.end());
    idx.insert(idx.end(), tix.begin(), tix.end());
  }
  // Launches of at most kIlvInlineTensors huff_ilv tensors take their
  // descriptors in the kernel arguments; the others read them from one
  // upload: [tensor descriptors][launch index arrays].  The status words are
  // host-coherent: zeroed here, ORed by the kernels, read after the stream
  // has drained (no copy back).
  PTWM_HIP_TRY(ctx.h_ilv_status.ensure(nt * sizeof(uint32_t)));
  uint32_t* const hs = static_cast<uint32_t*>(ctx.h_ilv_status.ptr);
  std::memset(hs, 0, nt * sizeof(uint32_t));
  auto inline_ok = [](const Launch& L) { return L.family == kFamilyHuff && L.m <= kIlvInlineTensors; };
  bool upload = false;
  for (const Launch& L : launches) upload |= !inline_ok(L);
  const size_t off_idx = align_up(nt * sizeof(IlvTensor), 16);
  const size_t args_bytes = off_idx + idx.size() * sizeof(uint32_t);
  uint8_t* d = nullptr;
  if (upload) {
    PTWM_HIP_TRY(ctx.ilv_args.ensure(args_bytes));
    PTWM_HIP_TRY(ctx.h_ilv.ensure(args_bytes));
    uint8_t* h = static_cast<uint8_t*>(ctx.h_ilv.ptr);
    std::memcpy(h, tensors.data(), nt * sizeof(IlvTensor));
    std::memcpy(h + off_idx, idx.data(), idx.size() * sizeof(uint32_t));
    d = static_cast<uint8_t*>(ctx.ilv_args.ptr);
    PTWM_HIP_TRY(hipMemcpyAsync(d, h, args_bytes, hipMemcpyHostToDevice, s));
  }
  if (ctx.profile) {
    PTWM_HIP_TRY(ctx.ensure_events());
    PTWM_HIP_TRY(hipEventRecord(ctx.ev[3], s));
  }
  const uint32_t* crc_tab = nullptr;
  for (const Launch& L : launches)
    if (L.crc && !crc_tab)
      if (int64_t rc = crc_tables(ctx, &crc_tab); rc != kOk) return rc;
  for (const Launch& L : launches) {
    const uint32_t* hidx = idx.data() + L.first;  // [m + 1 prefix][m tensor indexes]
    if (inline_ok(L)) {
      IlvInline inl{};
      inl.m = L.m;
      for (uint32_t j = 0; j <= L.m; ++j) inl.tpre[j] = hidx[j];
      for (uint32_t j = 0; j < L.m; ++j) {
        inl.tix[j] = hidx[L.m + 1 + j];
        inl.t[j] = tensors[inl.tix[j]];
      }
      PTWM_HIP_TRY(launch_ilv_decode(L.chain, nullptr, nullptr, nullptr, 0, inl, L.grid, hs, L.slots,
                                     L.stage_words, L.crc ? crc_tab : nullptr,
                                     static_cast<uint32_t*>(ctx.crc_part.ptr), s));
      continue;
    }
    const uint32_t* base = reinterpret_cast<const uint32_t*>(d + off_idx) + L.first;
    const IlvTensor* td = reinterpret_cast<const IlvTensor*>(d);
    if (L.family == kFamilyHuff)
      PTWM_HIP_TRY(launch_ilv_decode(L.chain, td, base + L.m + 1, base, L.m, IlvInline{}, L.grid, hs, L.slots,
                                     L.stage_words, L.crc ? crc_tab : nullptr,
                                     static_cast<uint32_t*>(ctx.crc_part.ptr), s));
    else
      PTWM_HIP_TRY(launch_rilv_decode(L.chain, td, base + L.m + 1, base, L.m, L.grid, hs, L.slots,
                                      L.stage_words, s));
  }
  if (ctx.profile) PTWM_HIP_TRY(hipEventRecord(ctx.ev[2], s));
  PTWM_HIP_TRY(hipStreamSynchronize(s));
  if (ctx.profile) {
    float ms = 0;
    PTWM_HIP_TRY(hipEventElapsedTime(&ms, ctx.ev[3], ctx.ev[2]));
    ctx.last_ms[0] += ms;
    ctx.last_ms[2] += ms;
  }
  std::vector<IlvTensor> again;
  for (size_t i = 0; i < nt; ++i) {
    if (hs[i] & ~kIlvRetrySlots) return kInvalidInput;
    if (hs[i]) again.push_back(tensors[i]);
  }
  if (!again.empty()) {
    if (all_slots) return kInternal;
    return ilv_decode_tensors(ctx, again, true);
  }
  return kOk;
}

}  // namespace ptwm
