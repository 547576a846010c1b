// rans_host.hip -- host orchestration of the rans_ilv encoder.
//
// Per call, any number of planes: histogram kernel (shared with huff_ilv) ->
// host normalisation (the reference's normalize_freqs) -> size kernel (word
// counts per block) -> host layout and header / offset-table uploads ->
// write kernel.  Each plane takes the smallest payload form
// (ilv_choose_form): coded, packed nibbles or stored.  Decode runs through ilv_decode_tensors (family
// kFamilyRans).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <vector>

#include "huffman_host.h"
#include "ilv_host.h"
#include "rans_ilv.h"
#include "runtime.h"

namespace ptwm {

static inline uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

int64_t rilv_encode_planes(DevCtx& ctx, const uint64_t* src, const uint64_t* n, uint32_t np, uint64_t out_dev,
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
  PTWM_HIP_TRY(hipMemcpyAsync(ctx.enc_planes.ptr, hp.data(), np * sizeof(IlvEncPlane), hipMemcpyHostToDevice, s));
  PTWM_HIP_TRY(hipMemsetAsync(ctx.enc_hist.ptr, 0, np * 256 * sizeof(uint32_t), s));
  PTWM_HIP_TRY(launch_ilv_hist(static_cast<const IlvEncPlane*>(ctx.enc_planes.ptr), np, max_n,
                               static_cast<uint32_t*>(ctx.enc_hist.ptr), s));
  std::vector<uint32_t> hist(np * 256);
  PTWM_HIP_TRY(hipMemcpyAsync(hist.data(), ctx.enc_hist.ptr, np * 256 * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
  PTWM_HIP_TRY(hipStreamSynchronize(s));
  // ---- frequency tables: per symbol f | cum << 16; headers ----
  std::vector<uint32_t> syms(np * 256, 0);
  std::vector<std::vector<uint8_t>> header(np);
  std::vector<bool> codable(np, false);
  for (uint32_t p = 0; p < np; ++p) {
    if (n[p] == 0) continue;
    uint16_t f[256], cum[256];
    int max_sym = 0;
    if (!rans_normalize_freqs(&hist[256 * p], f, cum, &max_sym)) continue;
    for (int sy = 0; sy < 256; ++sy) syms[256 * p + sy] = (uint32_t)f[sy] | ((uint32_t)cum[sy] << 16);
    std::vector<uint8_t>& h = header[p];
    h.push_back((uint8_t)max_sym);
    for (int i = 0; i <= max_sym; ++i) {
      h.push_back((uint8_t)f[i]);
      h.push_back((uint8_t)(f[i] >> 8));
    }
    codable[p] = true;
  }
  // ---- size pass over every block of every codable plane ----
  std::vector<RilvEncBlock> blocks;
  std::vector<uint32_t> first_block(np, 0), nbs(np, 0);
  for (uint32_t p = 0; p < np; ++p) {
    first_block[p] = (uint32_t)blocks.size();
    if (!codable[p]) continue;
    nbs[p] = (uint32_t)((n[p] + kIlvBlock - 1) / kIlvBlock);
    for (uint32_t b = 0; b < nbs[p]; ++b) blocks.push_back(RilvEncBlock{0, p, b});
  }
  const uint32_t nblk = (uint32_t)blocks.size();
  std::vector<uint32_t> bwords(nblk);
  if (nblk) {
    PTWM_HIP_TRY(ctx.enc_codes.ensure(syms.size() * sizeof(uint32_t)));
    PTWM_HIP_TRY(ctx.enc_blocks.ensure(nblk * sizeof(RilvEncBlock)));
    PTWM_HIP_TRY(ctx.enc_block_bytes.ensure(nblk * sizeof(uint32_t)));
    PTWM_HIP_TRY(hipMemcpyAsync(ctx.enc_codes.ptr, syms.data(), syms.size() * 4, hipMemcpyHostToDevice, s));
    PTWM_HIP_TRY(
        hipMemcpyAsync(ctx.enc_blocks.ptr, blocks.data(), nblk * sizeof(RilvEncBlock), hipMemcpyHostToDevice, s));
    PTWM_HIP_TRY(launch_rilv_size(static_cast<const IlvEncPlane*>(ctx.enc_planes.ptr),
                                  static_cast<const RilvEncBlock*>(ctx.enc_blocks.ptr), nblk,
                                  static_cast<const uint32_t*>(ctx.enc_codes.ptr),
                                  static_cast<uint32_t*>(ctx.enc_block_bytes.ptr), s));
    PTWM_HIP_TRY(hipMemcpyAsync(bwords.data(), ctx.enc_block_bytes.ptr, nblk * 4, hipMemcpyDeviceToHost, s));
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
      for (uint32_t b = 0; b < nbs[p]; ++b) d += align_up(kRilvBlockHead + 2ull * bwords[first_block[p] + b], 4);
      head[p] = align_up(5 + header[p].size(), 4);
      pay = head[p] + 4ull * (nbs[p] + 1) + d;
      codable_p = d <= 0xFFFFFFFFull;
    }
    form[p] = ilv_choose_form(n[p], all_nibbles(&hist[256 * p]), codable_p, pay, identity_fallback, &res[p].len);
    res[p].coded = form[p] == kFormCoded ? 1 : 0;
    res[p].codec = form[p] == kFormIdentity ? kCodecIdentity : kCodecRansIlv;
    off += res[p].len;
  }
  const uint64_t total = off;
  if (total > out_cap) {
    if (needed) *needed = total;
    return kBufferTooSmall;
  }
  // ---- headers, offset tables, stored / packed planes; block destinations ----
  // (host buffers of the asynchronous uploads stay alive until the final
  // stream synchronisation)
  std::vector<uint8_t> keep;
  if (int64_t rc = ilv_store_planes(ctx, src, n, np, out_dev, res, form.data(), keep); rc != kOk) return rc;
  std::vector<std::vector<uint8_t>> hbufs(np);
  std::vector<RilvEncBlock> live;
  std::vector<uint32_t> lw;
  for (uint32_t p = 0; p < np; ++p) {
    const uint64_t dst = out_dev + res[p].offset;
    if (!res[p].coded) continue;
    std::vector<uint8_t>& hbuf = hbufs[p];
    hbuf.assign(head[p] + 4ull * (nbs[p] + 1), 0);
    hbuf[0] = 1;
    const uint32_t nn = (uint32_t)n[p];
    std::memcpy(hbuf.data() + 1, &nn, 4);
    std::memcpy(hbuf.data() + 5, header[p].data(), header[p].size());
    uint32_t* tab = reinterpret_cast<uint32_t*>(hbuf.data() + head[p]);
    uint64_t acc = 0;
    const uint64_t data_dev = dst + hbuf.size();
    for (uint32_t b = 0; b < nbs[p]; ++b) {
      tab[b] = (uint32_t)acc;
      RilvEncBlock bk = blocks[first_block[p] + b];
      bk.dst = data_dev + acc;
      live.push_back(bk);
      acc += align_up(kRilvBlockHead + 2ull * bwords[first_block[p] + b], 4);
    }
    tab[nbs[p]] = (uint32_t)acc;
    PTWM_HIP_TRY(hipMemcpyAsync(reinterpret_cast<void*>(dst), hbuf.data(), hbuf.size(), hipMemcpyHostToDevice, s));
  }
  if (!live.empty()) {
    // block word counts in the order of `live`
    for (const RilvEncBlock& bk : live) lw.push_back(bwords[first_block[bk.plane] + bk.block]);
    PTWM_HIP_TRY(ctx.enc_lane_words.ensure(lw.size() * 4));
    PTWM_HIP_TRY(hipMemcpyAsync(ctx.enc_lane_words.ptr, lw.data(), lw.size() * 4, hipMemcpyHostToDevice, s));
    PTWM_HIP_TRY(
        hipMemcpyAsync(ctx.enc_blocks.ptr, live.data(), live.size() * sizeof(RilvEncBlock), hipMemcpyHostToDevice, s));
    PTWM_HIP_TRY(launch_rilv_encode(static_cast<const IlvEncPlane*>(ctx.enc_planes.ptr),
                                    static_cast<const RilvEncBlock*>(ctx.enc_blocks.ptr), (uint32_t)live.size(),
                                    static_cast<const uint32_t*>(ctx.enc_codes.ptr),
                                    static_cast<const uint32_t*>(ctx.enc_lane_words.ptr), s));
  }
  PTWM_HIP_TRY(hipStreamSynchronize(s));
  return (int64_t)total;
}

}  // namespace ptwm
