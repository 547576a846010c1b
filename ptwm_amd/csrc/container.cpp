// container.cpp -- the reference's three file layouts read into a decode plan.
//
// A .ptwm file is opened on the host (this file: plain C++, no device code)
// and turned into a PTMD plan whose payload offsets index the file's own
// bytes, so the caller copies the file to the device once and restores every
// tensor with one ptwm_hardware_backend_v1_dispatch_decode_cuda call.
//
//   legacy  \x89PTWM / \x89PTWX  container.rs:1590-1790 (open), header.rs,
//                                extension/table.rs, prelude.rs,
//                                chain/wire.rs, tensor_record.rs:265-420,
//                                plane_record.rs:110-272, index.rs
//   compact \x89PTWC             ptwc.rs:105-298, extension/compact_table.rs,
//                                tensor_record_compact.rs:497-815,
//                                chain/wire_compact.rs
//   frame   \x89PTWS             compact.rs:321-550 (one tensor)
//
// Per tensor the reader resolves the chain and recognises the shapes the
// device decodes (the fused pairs of chain/runtime.rs:744-826 and the
// one-op chains), maps each plane's codec through the Extension Table entry
// it names, and carries the plane CRC-32s, the chunk tables and the payload
// hash into the plan.  The plane lengths follow from orig_size through the
// chain, as the reference's inverse must reproduce orig_size
// (container.rs:2167-2175).  A tensor the device path does not take (another
// chain, a codec without a device decoder, shared codec state) is listed
// with status -5 so that the caller decodes it another way; a record that
// the reference rejects when it decodes it is listed with -1.  Errors in the
// file's own sections (header, tables, registry, index) fail the whole call
// with -1, as opening the container fails there.
//
// Checks the reference makes that this reader does not: the legacy
// Extension Table's BLAKE3 (a trust check over metadata the plan does not
// use), the re-derivation of built-in canonical ids from their labels, and
// the canonical-form rejections of the compact layouts (minimal
// encodings are still required of varints).
#include <algorithm>
#include <array>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/ptwm_mi355x.h"
#include "blake3_host.h"
#include "dtype_codes.h"
#include "xxh64_host.h"

namespace ptwm {
namespace {

constexpr int64_t kOk = 0, kInvalid = -1, kUnsup = -5;

// OpId wire ids (transforms/op.rs:11-36)
enum : uint16_t {
  kOpSource = 0x0000,
  kOpBitReorderIeee16 = 0x0010,
  kOpBitReorderIeee32 = 0x0011,
  kOpBitReorderE4M3 = 0x0012,
  kOpBitReorderE5M2 = 0x0013,
  kOpByteSplit = 0x0020,
  kOpNibbleSplit = 0x0021,
  kOpBytePassthrough = 0x0030,
  kOpIntDelta = 0x0052,
  kOpPredictorXor = 0x0053,
  kOpMantissaZeroStrip = 0x0064,
};

struct NamedId {
  const char* name;
  uint16_t id;
};
// transforms/op.rs:73-99 (names) with the wire ids of op.rs:11-36
const NamedId kOpNames[] = {
    {"source", 0x0000},          {"terminal", 0x0001},          {"bit_reorder_ieee16", 0x0010},
    {"bit_reorder_ieee32", 0x0011}, {"bit_reorder_fp8_e4m3", 0x0012}, {"bit_reorder_fp8_e5m2", 0x0013},
    {"byte_split", 0x0020},      {"nibble_split", 0x0021},      {"byte_passthrough", 0x0030},
    {"mxfp4_deinterleave", 0x0040}, {"block_microscaling_repack", 0x0041}, {"xor_delta", 0x0050},
    {"float_delta", 0x0051},     {"int_delta", 0x0052},         {"predictor_xor", 0x0053},
    {"index_bitwidth_pack", 0x0060}, {"entropy_estimate", 0x0061}, {"concat", 0x0062},
    {"reshape", 0x0063},         {"mantissa_zero_strip", 0x0064}, {"burrows_wheeler", 0x0070},
    {"move_to_front", 0x0071},   {"spherical_normalize", 0x0080}, {"alpha_stable_normalize", 0x0081},
};
// codec.rs:28-46 (REGISTRY)
const NamedId kCodecNames[] = {
    {"identity", 0x0000},       {"huffman", 0x0001},           {"huffman_nibble", 0x0002},
    {"rans", 0x0003},           {"zstd", 0x0004},              {"zstd_dict", 0x0005},
    {"fpc", 0x0006},            {"tans", 0x0007},              {"per_group_codebook", 0x0010},
    {"order1_scale_ac", 0x0011}, {"arithmetic_o0", 0x0012},    {"arithmetic_o0_adaptive", 0x0013},
    {"arithmetic_o1", 0x0014},  {"context_mixing_lite", 0x0015}, {"huff_llm_5bit", 0x0016},
    {"order1_arithmetic", 0x0017}, {"neural_predictor", 0x0018},
};

// Built-ins with an Extension Table entry but no wire id (extension/
// builtins.rs BUILTIN_SPECS: the host-side chain builder and classifiers):
// the only names a compact table stores under its named tag.
const char* const kNamedOnly[] = {"production_chains", "classifier_heuristic", "classifier_hf_quant_config",
                                  "classifier_ptwm_config", "classifier_explicit_flags"};
// The built-in names: these five, the ops and the codecs above (all of
// BUILTIN_SPECS, plus huffman_nibble, which has a wire id but no entry).
constexpr const char* kBuiltinVersion = "1.1.0";  // CURRENT_BUILTIN_VERSION (the crate version)

// CanonicalId::derive (extension/id.rs:21-30) with the built-ins' author key
// (extension/mod.rs BUILTIN_PUBKEY, 32 bytes of 0xBB)
void builtin_id(const std::string& name, const std::string& ver, uint8_t out[32]) {
  std::vector<uint8_t> pre(32, 0xBB);
  pre.push_back(0);
  pre.insert(pre.end(), name.begin(), name.end());
  pre.push_back(0);
  pre.insert(pre.end(), ver.begin(), ver.end());
  blake3_hash(pre.data(), pre.size(), out);
}

// The built-in an Extension Table entry names, as the reference dispatches
// it (extension/builtins.rs:302-332 normalize_builtin_ids, then the registry
// by id): an id of a built-in at the current version, or a built-in label
// "io.ptwm.builtin.<name>@<version>" of another valid version whose id is
// that version's derivation.  Returns the name, or empty.
std::string builtin_of(const uint8_t* id, const uint8_t* label, size_t ll) {
  struct CurrentIds {
    std::vector<std::pair<std::string, std::array<uint8_t, 32>>> ids;
    CurrentIds() {
      std::vector<std::string> names;
      for (const NamedId& n : kOpNames) names.push_back(n.name);
      for (const NamedId& n : kCodecNames) names.push_back(n.name);
      for (const char* n : kNamedOnly) names.push_back(n);
      for (const std::string& n : names) {
        std::array<uint8_t, 32> a;
        builtin_id(n, kBuiltinVersion, a.data());
        ids.emplace_back(n, a);
      }
    }
  };
  static const CurrentIds cur;
  for (const auto& e : cur.ids)
    if (std::memcmp(e.second.data(), id, 32) == 0) return e.first;
  static const char kPrefix[] = "io.ptwm.builtin.";
  const size_t pl = sizeof(kPrefix) - 1;
  if (ll <= pl || std::memcmp(label, kPrefix, pl) != 0) return std::string();
  const std::string rest(reinterpret_cast<const char*>(label) + pl, ll - pl);
  const size_t at = rest.find('@');
  if (at == std::string::npos) return std::string();
  const std::string name = rest.substr(0, at), ver = rest.substr(at + 1);
  // is_valid_builtin_version: non-empty, at most 64 bytes, no '@'
  if (ver.empty() || ver.size() > 64 || ver.find('@') != std::string::npos || ver == kBuiltinVersion)
    return std::string();
  bool known = false;  // a name with an entry (BuiltinRegistry::by_name)
  for (const auto& e : cur.ids) known |= e.first == name && name != "huffman_nibble";
  if (!known) return std::string();
  uint8_t want[32];
  builtin_id(name, ver, want);
  return std::memcmp(want, id, 32) == 0 ? name : std::string();
}

bool known_op(uint64_t id) {
  for (const NamedId& n : kOpNames)
    if (n.id == id) return true;
  return false;
}
bool known_codec(uint64_t id) {
  for (const NamedId& n : kCodecNames)
    if (n.id == id) return true;
  return false;
}

// Plane codecs the device decode takes (runtime.hip parse_plan).
constexpr uint16_t kHuffIlv = 0x7F01, kRansIlv = 0x7F02;
constexpr uint16_t kO1sac = 0x0011;  // Order1ScaleAC (codecs/order1_scale_ac.rs)
bool device_codec(uint16_t c) {
  return c == 0x0000 || c == 0x0001 || c == 0x0003 || c == 0x0004 || c == 0x0007 || c == kO1sac || c == kHuffIlv ||
         c == kRansIlv;
}

// This library's own plane codec contributions (blake3 ids of
// extension/id.rs:21-30 with the all-zero author key).
const uint8_t kOwnHuffIlvId[32] = {0xcf, 0xd8, 0xcc, 0x03, 0x48, 0x3e, 0xb4, 0xa4, 0x3c, 0xdd, 0xdb,
                                   0x4b, 0x3c, 0xbf, 0x95, 0xb3, 0x2e, 0xa0, 0xf3, 0x0e, 0x17, 0xe5,
                                   0xec, 0x85, 0xa0, 0xb5, 0x2d, 0xe0, 0x4e, 0x8c, 0xaf, 0x04};
const uint8_t kOwnRansIlvId[32] = {0x96, 0x8f, 0x8b, 0xe9, 0xf0, 0x6b, 0x14, 0xb5, 0x3f, 0xcd, 0x06,
                                   0x66, 0x22, 0x49, 0x3f, 0x11, 0x01, 0x95, 0x4d, 0x07, 0x4d, 0x25,
                                   0xd6, 0x3e, 0x78, 0x38, 0x0f, 0xe5, 0x3e, 0x1f, 0xf1, 0xf5};

// ---- byte cursor over one section --------------------------------------

struct Rd {
  const uint8_t* b;
  size_t n;
  size_t o = 0;
  bool ok = true;
  // a section whose bytes could not be taken (null) reads as truncated
  Rd(const uint8_t* p, size_t len) : b(p), n(p ? len : 0), ok(p != nullptr || len == 0) {}
  size_t left() const { return ok ? n - o : 0; }
  const uint8_t* take(size_t k) {
    if (!ok || n - o < k) {
      ok = false;
      return nullptr;
    }
    const uint8_t* p = b + o;
    o += k;
    return p;
  }
  uint64_t le(int bytes) {
    const uint8_t* p = take((size_t)bytes);
    uint64_t v = 0;
    if (p)
      for (int i = bytes - 1; i >= 0; --i) v = (v << 8) | p[i];
    return v;
  }
  uint8_t u8() { return (uint8_t)le(1); }
  uint16_t u16() { return (uint16_t)le(2); }
  uint32_t u32() { return (uint32_t)le(4); }
  uint64_t u64() { return le(8); }
  // canonical unsigned LEB128 of at most 10 bytes (varint.rs:40-62)
  uint64_t var() {
    uint64_t v = 0;
    for (int i = 0; i < 10; ++i) {
      if (!ok || o >= n) {
        ok = false;
        return 0;
      }
      const uint8_t c = b[o++];
      if (i == 9 && c > 1) {
        ok = false;
        return 0;
      }
      v |= (uint64_t)(c & 0x7F) << (7 * i);
      if (!(c & 0x80)) {
        if (i > 0 && c == 0) ok = false;  // non-minimal
        return ok ? v : 0;
      }
    }
    ok = false;
    return 0;
  }
  uint64_t var_max(uint64_t mx) {
    uint64_t v = var();
    if (v > mx) ok = false;
    return ok ? v : 0;
  }
  // a varint length that must fit in what is left (Cursor::len_varint)
  size_t var_len() {
    uint64_t v = var();
    if (!ok || v > left()) {
      ok = false;
      return 0;
    }
    return (size_t)v;
  }
  bool done() const { return ok && o == n; }
};

// std::str::from_utf8: well-formed UTF-8 (no overlong forms, no surrogates,
// nothing above U+10FFFF)
bool valid_utf8(const uint8_t* p, size_t n) {
  for (size_t i = 0; i < n;) {
    const uint8_t c = p[i];
    if (c < 0x80) {
      ++i;
      continue;
    }
    size_t k;
    uint32_t lo = 0x80, hi = 0xBF;
    if (c >= 0xC2 && c <= 0xDF) k = 1;
    else if (c >= 0xE0 && c <= 0xEF) {
      k = 2;
      if (c == 0xE0) lo = 0xA0;
      if (c == 0xED) hi = 0x9F;
    } else if (c >= 0xF0 && c <= 0xF4) {
      k = 3;
      if (c == 0xF0) lo = 0x90;
      if (c == 0xF4) hi = 0x8F;
    } else {
      return false;
    }
    if (n - i <= k) return false;
    if (p[i + 1] < lo || p[i + 1] > hi) return false;
    for (size_t j = 2; j <= k; ++j)
      if ((p[i + j] & 0xC0) != 0x80) return false;
    i += k + 1;
  }
  return true;
}

// ---- chains --------------------------------------------------------------

struct Node {
  uint16_t op;
  bool bound;               // a CW2 Source whose params come from the tensor
  std::vector<uint8_t> params;
};
struct Edge {
  uint32_t src, src_out, dst, dst_in;
};
struct Term {
  uint32_t node, out;
};
struct Chain {
  std::vector<Node> nodes;
  std::vector<Edge> edges;
  std::vector<Term> terms;
};

// Extension Table entry, as far as the plan needs it.
struct EtEntry {
  int kind = 0;  // 0 other, 1 built-in op, 2 plane codec
  uint16_t id = 0;
  bool builtin = false;  // a built-in's entry (full-entry form only)
  bool wasm = false;     // carries an embedded WASM range (full-entry form only)
};

// Role::write bytes (types/role.rs:250-330): parsed for their length, with
// the value checks of Role::read (ScaleFormat 0..=4, NibbleKind 0..=2, the
// ValueFormat and ResidualFormat tags).  `coded`: whether the role has a
// one-byte compact code (chain/wire_compact.rs:439-462 role_code).
bool skip_role(Rd& r, bool* coded = nullptr) {
  const uint8_t t = r.u8();
  bool c = false;
  switch (t) {
    case 0x00: case 0x07: if (r.u8() > 4) r.ok = false; c = true; break;   // Scale / GlobalScale
    case 0x04: if (r.u8() > 2) r.ok = false; c = true; break;              // Nibble
    case 0x01: {                                                           // Value
      const uint8_t f = r.u8();
      if (f == 0) c = true;                                                // Fp4E2m1
      else if (f == 1) { const uint8_t bits = r.u8(); c = bits >= 1 && bits <= 32; }  // IntN
      else r.ok = false;
      break;
    }
    case 0x02: case 0x05: {                                                // MantissaByte / IntegerByte
      const uint8_t index = r.u8(), of = r.u8();
      c = index < of && of >= 1 && of <= 8;
      break;
    }
    case 0x03: case 0x08: case 0x09: c = true; break;                      // ExponentByte / Raw / Index
    case 0x06: {                                                           // Residual
      const uint8_t f = r.u8();
      if (f == 0) c = true;                                                // Xor
      else if (f == 1) r.u16();                                            // FloatDelta { dtype }
      else r.ok = false;
      break;
    }
    case 0xFF: { r.u16(); const uint16_t l = r.u16(); r.take(l); break; }  // Vendor
    default: r.ok = false;
  }
  if (coded) *coded = c;
  return r.ok;
}

// CW2 one-byte roles (chain/wire_compact.rs:485-535); an escaped role that
// has a one-byte code is not canonical
bool skip_compact_role(Rd& r) {
  const uint8_t b = r.u8();
  if (!r.ok) return false;
  if (b == 0xFF) {
    bool coded = false;
    if (!skip_role(r, &coded)) return false;
    if (coded) r.ok = false;
    return r.ok;
  }
  if (b <= 0x04 || (b >= 0x08 && b <= 0x0C) || (b >= 0x10 && b <= 0x12) || (b >= 0x18 && b <= 0x1C)) return true;
  if (b >= 0x40 && b < 0xC0) {  // MantissaByte / IntegerByte: 8 (of - 1) + index, index < of
    const uint32_t k = b & 0x3F, of = k / 8 + 1, index = k % 8;
    if (index >= of) r.ok = false;
    return r.ok;
  }
  if (b >= 0xC0 && b <= 0xDF) return true;  // Value { IntN { 1..=32 } }
  r.ok = false;
  return false;
}

// Legacy ExtensionTableEntry (extension/table.rs): canonical id, label, kind,
// abi, lifecycle, flavors, capabilities (u32 + CBOR, at most 1 MiB),
// attestation kind + u16 bytes, install hint, embedded WASM range.
bool read_legacy_entry(Rd& r, EtEntry& e) {
  const uint8_t* id = r.take(32);
  const uint16_t ll = r.u16();
  const uint8_t* label = r.take(ll);
  r.u16();  // kind
  r.u16();  // abi_version
  r.u8();   // lifecycle
  r.u8();   // flavor hints
  const uint32_t cl = r.u32();
  if (cl > (1u << 20)) r.ok = false;
  r.take(cl);
  r.u8();  // attestation kind
  r.take(r.u16());
  r.take(r.u16());  // install hint
  const uint64_t wasm_off = r.u64(), wasm_len = r.u64();  // embedded WASM offset / length
  if (!r.ok || !valid_utf8(label, ll)) return r.ok = false;
  e = EtEntry{};
  e.wasm = wasm_off != 0 || wasm_len != 0;
  if (std::memcmp(id, kOwnHuffIlvId, 32) == 0) {
    e.kind = 2;
    e.id = kHuffIlv;
    return true;
  }
  if (std::memcmp(id, kOwnRansIlvId, 32) == 0) {
    e.kind = 2;
    e.id = kRansIlv;
    return true;
  }
  const std::string name = builtin_of(id, label, ll);
  if (name.empty()) return true;  // a third-party entry
  e.builtin = true;
  for (const NamedId& n : kOpNames)
    if (name == n.name) {
      e.kind = 1;
      e.id = n.id;
    }
  for (const NamedId& n : kCodecNames)
    if (name == n.name) {
      e.kind = 2;
      e.id = n.id;
    }
  return true;
}

bool read_legacy_table(Rd& r, std::vector<EtEntry>& et) {
  const uint32_t count = r.u32();
  if (!r.ok || count > 65536u || count > r.left() / 32) return r.ok = false;
  et.assign(count, EtEntry{});
  for (uint32_t i = 0; i < count; ++i)
    if (!read_legacy_entry(r, et[i])) return false;
  return true;
}

// compact Extension Table (extension/compact_table.rs:242-261)
bool read_compact_table(const uint8_t* p, size_t n, std::vector<EtEntry>& et) {
  Rd r(p, n);
  const uint64_t count = r.var_max(1u << 16);
  if (!r.ok || count > n / 2) return false;
  et.assign((size_t)count, EtEntry{});
  for (size_t i = 0; i < count; ++i) {
    const uint8_t tag = r.u8();
    if (tag == 0x01) {
      const uint64_t id = r.var();
      if (!known_op(id)) return false;
      et[i].kind = 1;
      et[i].id = (uint16_t)id;
    } else if (tag == 0x02) {
      const uint64_t id = r.var();
      if (!known_codec(id)) return false;
      et[i].kind = 2;
      et[i].id = (uint16_t)id;
    } else if (tag == 0x03) {
      // extension/compact_table.rs:198-214: a built-in by name, allowed only
      // for the built-ins without a wire id (those use their tags)
      const uint64_t l = r.var();
      if (l < 1 || l > 255) return false;
      const uint8_t* nm = r.take((size_t)l);
      if (!r.ok) return false;
      bool named_only = false;
      for (const char* n : kNamedOnly) named_only |= std::strlen(n) == l && std::memcmp(n, nm, (size_t)l) == 0;
      if (!named_only) return false;
    } else if (tag == 0x7F) {
      // compact_table.rs:215-235: a third-party entry; a built-in's entry or
      // one with embedded WASM is refused
      const size_t l = r.var_len();
      Rd sub(r.take(l), l);
      if (!r.ok || !read_legacy_entry(sub, et[i]) || !sub.done()) return false;
      if (et[i].builtin || et[i].wasm) return false;
    } else {
      return false;
    }
    if (!r.ok) return false;
  }
  return r.done();
}

// legacy chain wire (chain/wire.rs): fixed-width counts and section lengths,
// ops as Extension Table indexes
bool read_legacy_chain(Rd& r, const std::vector<EtEntry>& et, Chain& c) {
  const uint32_t nn = r.u8(), ne = r.u8(), nt = r.u8();
  const uint16_t nl = r.u16(), el = r.u16(), tl = r.u16();
  Rd rn(r.take(nl), nl), re(r.take(el), el), rt(r.take(tl), tl);
  if (!r.ok) return false;
  c = Chain{};
  for (uint32_t i = 0; i < nn; ++i) {
    const uint16_t op = rn.u16();
    const uint8_t pl = rn.u8();
    const uint8_t* pp = rn.take(pl);
    if (!rn.ok) return false;
    if (op >= et.size() || et[op].kind != 1) return false;
    c.nodes.push_back(Node{et[op].id, false, std::vector<uint8_t>(pp, pp + pl)});
  }
  for (uint32_t i = 0; i < ne; ++i) {
    Edge e{re.u8(), re.u8(), re.u8(), re.u8()};
    if (re.u8() && !skip_role(re)) return false;
    re.take(re.u16());
    if (!re.ok) return false;
    c.edges.push_back(e);
  }
  for (uint32_t i = 0; i < nt; ++i) {
    Term t{rt.u8(), rt.u8()};
    if (!skip_role(rt)) return false;
    c.terms.push_back(t);
  }
  return rn.done() && re.done() && rt.done();
}

// CW2 (chain/wire_compact.rs:1-66).  op_is_wire: op_ref is the OpId wire id
// (PTWS frame), else an index into `et`.  A Source with no params is bound:
// it takes `binding` when one is given, else stays marked (registry chains).
bool read_cw2(Rd& r, bool op_is_wire, const std::vector<EtEntry>* et, const std::vector<uint8_t>* binding,
              bool defer, Chain& c) {
  c = Chain{};
  const uint64_t nn = r.var(), ne = r.var(), nt = r.var();
  if (!r.ok || nn < 1 || nn > 255 || ne > 255 || nt > 255) return false;
  for (uint64_t i = 0; i < nn; ++i) {
    const uint64_t ref = r.var();
    const uint64_t pl = r.var_max(255);
    const uint8_t* pp = r.take((size_t)pl);
    if (!r.ok) return false;
    uint16_t op;
    if (op_is_wire) {
      if (!known_op(ref)) return false;
      op = (uint16_t)ref;
    } else {
      if (ref >= et->size() || (*et)[ref].kind != 1) return false;
      op = (*et)[ref].id;
    }
    Node nd{op, false, std::vector<uint8_t>(pp, pp + pl)};
    if (op == kOpSource && pl == 0) {
      if (binding) {
        nd.params = *binding;
      } else if (defer) {
        nd.bound = true;
      } else {
        return false;  // a bound Source with no tensor shape to bind
      }
    } else if (op == kOpSource && binding && nd.params == *binding) {
      return false;  // explicit params equal to the binding (non-canonical)
    }
    c.nodes.push_back(std::move(nd));
  }
  uint64_t spine = 0;
  if (ne > 0) spine = r.var_max(ne);
  for (uint64_t i = 0; i < spine; ++i) c.edges.push_back(Edge{(uint32_t)i, 0, (uint32_t)i + 1, 0});
  for (uint64_t i = spine; i < ne; ++i) {
    Edge e{(uint32_t)r.var_max(255), (uint32_t)r.var_max(255), (uint32_t)r.var_max(255), (uint32_t)r.var_max(255)};
    const uint8_t etag = r.u8();
    if (!r.ok || (etag & ~3u)) return false;
    // the spine's next edge written out (no role, no vendor bytes) is not canonical
    if (i == spine && etag == 0 && e.src == i && e.src_out == 0 && e.dst == i + 1 && e.dst_in == 0) return false;
    if ((etag & 1u) && !skip_compact_role(r)) return false;
    if (etag & 2u) {
      const uint64_t vl = r.var();
      if (vl < 1 || vl > 65535) return false;
      r.take((size_t)vl);
    }
    if (!r.ok) return false;
    c.edges.push_back(e);
  }
  for (uint64_t i = 0; i < nt; ++i) {
    const uint8_t ref = r.u8();
    Term t{(uint32_t)(ref >> 4), (uint32_t)(ref & 15u)};
    if (ref == 0xFF) {  // escaped (node, output): only when the byte cannot hold them
      t = Term{r.u8(), r.u8()};
      if (t.node <= 14 && t.out <= 15) return false;
    } else if ((ref >> 4) == 15) {
      return false;  // reserved
    }
    if (!skip_compact_role(r)) return false;
    c.terms.push_back(t);
  }
  return r.ok;
}

// ---- Source params and widths (transforms/source.rs:14-130) -------------

int elem_bytes(uint16_t chain_dtype) {  // element_width_for, in bytes; 0 = nibble
  switch (chain_dtype) {
    case 0x0002: case 0x000F: case 0x0007: case 0x0008: return 2;
    case 0x0003: case 0x0009: case 0x000A: return 4;
    case 0x0004: case 0x000B: case 0x000C: return 8;
    case 0x001F: return 0;
    default: return 1;
  }
}

// Source length in bytes and its chain dtype (read_source_params +
// output_descriptor); false when the params do not parse or overflow.
bool source_len(const std::vector<uint8_t>& p, uint64_t& len, uint16_t& dtype) {
  if (p.empty()) return false;
  const size_t nd = p[0];
  if (p.size() < 1 + 4 * nd + 2) return false;
  unsigned __int128 n = 1;
  for (size_t i = 0; i < nd; ++i) {
    uint32_t d;
    std::memcpy(&d, p.data() + 1 + 4 * i, 4);
    n *= d;
    if (n > UINT64_MAX) return false;
  }
  dtype = (uint16_t)(p[1 + 4 * nd] | (p[2 + 4 * nd] << 8));
  const int eb = elem_bytes(dtype);
  n *= (eb == 0 ? 1 : eb);
  if (n > UINT64_MAX) return false;
  len = (uint64_t)n;
  return true;
}

// The fused chains of the decode plan (transforms/fusion.rs; PTMD ids).
enum : uint8_t { kPtmdIeee16 = 1, kPtmdIeee32 = 2, kPtmdE4M3 = 3, kPtmdE5M2 = 4, kPtmdNibble = 5, kPtmdPass = 6 };
int ptmd_planes(int ch) { return ch == kPtmdIeee32 ? 4 : ch == kPtmdPass ? 1 : 2; }
int ptmd_ratio(int ch) { return ch == kPtmdIeee16 ? 2 : ch == kPtmdIeee32 ? 4 : 1; }

// The production split chains with one plane op (python/ptwm/preprocessing/
// _chains.py:360-600): Source -> BitReorderIeee16|32 -> ByteSplit(2|4), and
// ByteSplit output j -> IntDelta | PredictorXor | MantissaZeroStrip(k) ->
// terminal, the other outputs terminals themselves.  Returns the PTMD chain
// (0: another shape, -1: the op's parameters are refused by
// chain/dispatch.rs:96-122), the terminal-to-plane map and op_flags[j], the
// PTMD plane flag bits of the op (byte elements: a ByteSplit output).
int recognise_plane_op(const Chain& c, std::vector<int>& perm, std::vector<uint32_t>& op_flags) {
  if (c.nodes.size() != 4 || c.nodes[0].op != kOpSource || c.edges.size() != 3) return 0;
  for (size_t i = 0; i < 2; ++i) {
    const Edge& e = c.edges[i];
    if (e.src != i || e.src_out != 0 || e.dst != i + 1 || e.dst_in != 0) return 0;
  }
  const Node& split = c.nodes[2];
  if (split.op != kOpByteSplit || split.params.size() != 1 || !c.nodes[1].params.empty()) return 0;
  int ch = 0;
  if (c.nodes[1].op == kOpBitReorderIeee16 && split.params[0] == 2) ch = kPtmdIeee16;
  else if (c.nodes[1].op == kOpBitReorderIeee32 && split.params[0] == 4) ch = kPtmdIeee32;
  if (!ch) return 0;
  const int np = split.params[0];
  const Edge& e = c.edges[2];
  if (e.src != 2 || e.src_out >= (uint32_t)np || e.dst != 3 || e.dst_in != 0) return 0;
  const Node& op = c.nodes[3];
  uint32_t flags = 0;
  if (op.op == kOpIntDelta || op.op == kOpPredictorXor) {
    if (!op.params.empty()) return -1;  // expect_empty_params
    flags = (op.op == kOpIntDelta ? 1u : 2u) << 1;  // element width 1: code 0
  } else if (op.op == kOpMantissaZeroStrip) {
    if (op.params.empty() || op.params[0] < 1 || op.params[0] > 7) return -1;  // MantissaZeroStrip::new
    flags = (3u << 1) | ((uint32_t)op.params[0] << 3);
  } else {
    return 0;
  }
  if ((int)c.terms.size() != np) return 0;
  perm.assign((size_t)np, -1);
  std::vector<char> seen((size_t)np, 0);
  for (int k = 0; k < np; ++k) {
    const Term& t = c.terms[(size_t)k];
    uint32_t q;
    if (t.node == 3 && t.out == 0) q = e.src_out;
    else if (t.node == 2 && t.out < (uint32_t)np && t.out != e.src_out) q = t.out;
    else return 0;
    if (seen[q]) return 0;
    seen[q] = 1;
    perm[(size_t)k] = (int)q;
  }
  op_flags.assign((size_t)np, 0);
  op_flags[e.src_out] = flags;
  return ch;
}

// Recognise a chain the device restores.  Returns the PTMD chain (0: none,
// -1: refused by the reference), per terminal the plane of that chain it
// carries, and per plane the PTMD plane-op flag bits.
int recognise(const Chain& c, std::vector<int>& perm, std::vector<uint32_t>& op_flags) {
  const size_t nn = c.nodes.size();
  op_flags.clear();
  if (nn == 0 || c.nodes[0].op != kOpSource) return 0;
  if (nn == 4) return recognise_plane_op(c, perm, op_flags);
  for (size_t i = 1; i < nn; ++i)
    if (!c.nodes[i].params.empty() && c.nodes[i].op != kOpByteSplit) return 0;
  // the node chain must be the spine 0 -> 1 -> ... (one input each)
  if (c.edges.size() != nn - 1) return 0;
  for (size_t i = 0; i + 1 < nn; ++i) {
    const Edge& e = c.edges[i];
    if (e.src != i || e.src_out != 0 || e.dst != i + 1 || e.dst_in != 0) return 0;
  }
  int ch = 0;
  const auto op = [&](size_t i) { return c.nodes[i].op; };
  const auto split_n = [&](size_t i) {
    return c.nodes[i].params.size() == 1 ? (int)c.nodes[i].params[0] : -1;
  };
  if (nn == 3) {
    if (op(1) == kOpBitReorderIeee16 && op(2) == kOpByteSplit && split_n(2) == 2) ch = kPtmdIeee16;
    else if (op(1) == kOpBitReorderIeee32 && op(2) == kOpByteSplit && split_n(2) == 4) ch = kPtmdIeee32;
    else if (op(1) == kOpBitReorderE4M3 && op(2) == kOpNibbleSplit) ch = kPtmdE4M3;
    else if (op(1) == kOpBitReorderE5M2 && op(2) == kOpNibbleSplit) ch = kPtmdE5M2;
  } else if (nn == 2) {
    if (op(1) == kOpNibbleSplit) ch = kPtmdNibble;
    else if (op(1) == kOpBytePassthrough) ch = kPtmdPass;
  } else if (nn == 1) {
    ch = kPtmdPass;  // a bare Source: its output is the tensor
  }
  if (!ch) return 0;
  const int np = ptmd_planes(ch);
  op_flags.assign((size_t)np, 0);
  if ((int)c.terms.size() != np) return 0;
  perm.assign((size_t)np, -1);
  std::vector<char> seen((size_t)np, 0);
  for (int k = 0; k < np; ++k) {
    const Term& t = c.terms[(size_t)k];
    if (t.node != nn - 1 || t.out >= (uint32_t)np || seen[t.out]) return 0;
    seen[t.out] = 1;
    perm[(size_t)k] = (int)t.out;
  }
  return ch;
}

// the op widths the fused chain's ops require of the Source
bool width_ok(int ch, uint16_t src_dtype) {
  const int eb = elem_bytes(src_dtype);
  switch (ch) {
    case kPtmdIeee16: return eb == 2;
    case kPtmdIeee32: return eb == 4;
    case kPtmdE4M3: case kPtmdE5M2: return eb == 1;
    case kPtmdNibble: return eb != 0;
    default: return true;
  }
}

// ---- records -------------------------------------------------------------

struct PlaneRec {
  uint16_t codec = 0;   // resolved through the Extension Table
  int et_kind = 0;
  uint8_t role = 0;
  uint8_t state_source = 0;
  uint8_t state_version = 0;
  uint16_t state_info = 0;                // shared state id (state_source 2)
  uint64_t inl_off = 0, inl_len = 0;      // inline state bytes (absolute file offsets)
  uint32_t row_len = 0;                   // plane layout: 0 Flat, else Rows { row_len }
  uint64_t payload_off = 0, payload_len = 0;  // absolute file offsets
  bool has_crc = false;
  uint32_t crc = 0;
  bool chunked = false;
  std::vector<uint32_t> chunks;  // (offset, size) pairs
};

struct TensorRec {
  uint64_t name_off = 0;
  uint32_t name_len = 0;
  uint64_t rec_off = 0, rec_len = 0;
  uint16_t dtype = 0;
  uint8_t input_format = 0;
  uint64_t orig = 0;
  bool has_hash = false;
  uint64_t hash = 0;
  const Chain* chain = nullptr;
  Chain own_chain;                // inline chain, or a registry chain bound to this record
  std::vector<PlaneRec> planes;
  int32_t status = 0;
};

// PlaneRole::from_u8 (types/plane_role.rs:12-40)
bool known_role(uint8_t r) { return (r >= 1 && r <= 6) || (r >= 0x10 && r <= 0x13); }

// legacy plane record (plane_record.rs:110-272); base = file offset of r's start
bool read_legacy_plane(Rd& r, uint64_t base, const std::vector<EtEntry>& et, PlaneRec& p) {
  const uint8_t role = r.u8();
  const uint8_t flags = r.u8();
  const uint16_t codec_raw = r.u16();
  const uint16_t cti = r.u16();
  p.role = role;
  p.state_source = r.u8();
  p.state_version = r.u8();
  p.state_info = r.u16();
  const uint32_t isl = r.u32();
  p.payload_len = r.u64();
  if (!r.ok || !known_role(role) || !known_codec(codec_raw) || p.state_source > 3) return r.ok = false;
  if (flags & 2u) {
    p.has_crc = true;
    p.crc = r.u32();
  }
  if (flags & 1u) {
    const uint32_t nc = r.u32();
    if (!r.ok || nc > r.left() / 8) return r.ok = false;
    p.chunked = true;
    p.chunks.resize(2 * (size_t)nc);
    for (uint32_t k = 0; k < 2 * nc; ++k) p.chunks[k] = r.u32();
  }
  if (p.state_source == 3) {  // external state reference
    r.u8();
    const uint8_t rf = r.u8();
    r.take(r.u16());
    r.u8();
    if (rf & 1u) r.take(32);
  }
  const uint8_t layout = r.u8();
  if (layout == 1) {
    p.row_len = r.u32();
    if (p.row_len == 0) r.ok = false;
  } else if (layout != 0) {
    r.ok = false;
  }
  p.inl_off = base + r.o;
  p.inl_len = isl;
  r.take(isl);
  if (!r.ok || p.payload_len > r.left()) return r.ok = false;
  p.payload_off = base + r.o;
  r.take((size_t)p.payload_len);
  if (cti >= et.size()) return r.ok = false;
  p.et_kind = et[cti].kind;
  p.codec = et[cti].id;
  return r.ok;
}

// One shared-state prelude entry (prelude.rs:5-20): the state bytes stay in
// the file, at [off, off + len).
struct PreludeEnt {
  uint16_t id = 0, codec = 0;
  uint8_t version = 0, mask = 0;
  uint64_t hash = 0;
  uint64_t off = 0, len = 0;
};

// parse_prelude (prelude.rs:65-150); base = file offset of r's start
// canonical: the compact container's prelude, whose reserved field and name
// padding must be zero (container.rs:1569-1580: one encoding per prelude)
bool read_prelude(Rd& r, uint64_t base, std::vector<PreludeEnt>& out, bool canonical = false) {
  const uint32_t pc = r.u32();
  if (!r.ok || pc > r.left() / 22) return false;  // MIN_ENTRY_BYTES
  out.clear();
  for (uint32_t i = 0; i < pc; ++i) {
    PreludeEnt e;
    e.id = r.u16();
    e.codec = r.u16();
    e.version = r.u8();
    e.mask = r.u8();
    const uint16_t reserved = r.u16();
    e.hash = r.u64();
    const uint16_t nl = r.u16();
    const uint8_t* name = r.take(nl);
    if (!r.ok || !known_codec(e.codec) || !valid_utf8(name, nl)) return false;
    const uint8_t* pad = r.take((4 - nl % 4) % 4);
    if (canonical && r.ok) {
      if (reserved != 0) return false;
      for (size_t k = 0; k < (4 - nl % 4) % 4u; ++k)
        if (pad[k] != 0) return false;
    }
    e.len = r.u32();
    e.off = base + r.o;
    r.take((size_t)e.len);
    if (!r.ok) return false;
    out.push_back(e);
  }
  return true;
}

// ---- plan assembly ---------------------------------------------------------

void put(std::vector<uint8_t>& v, uint64_t x, int bytes) {
  for (int i = 0; i < bytes; ++i) v.push_back((uint8_t)(x >> (8 * i)));
}

constexpr uint64_t kOutAlign = 256;

struct Builder {
  std::vector<uint8_t> plan;
  uint32_t n_plan = 0;
  uint64_t out_len = 0;
  bool strict = false;  // compact layouts: Source length == orig_size
  const uint8_t* file = nullptr;
  std::vector<PreludeEnt> prelude;
  Builder() { put(plan, 0x444D5450u, 4), put(plan, 1, 2), put(plan, 0, 2), put(plan, 0, 4); }

  // status of one tensor; appends its plan entry when planned
  int32_t add(TensorRec& t, uint8_t& chain_out, uint64_t& out_off, int32_t& plan_index, uint32_t& info_flags) {
    chain_out = 0;
    plan_index = -1;
    out_off = 0;
    info_flags = (t.has_hash ? 1u : 0u);
    if (!t.chain) return kInvalid;
    const Chain& c = *t.chain;
    // container.rs:1846-1868: the Source bounds the tensor
    if (c.nodes.empty() || c.nodes[0].op != kOpSource || c.nodes[0].bound) return kInvalid;
    uint64_t slen = 0;
    uint16_t sdt = 0;
    if (!source_len(c.nodes[0].params, slen, sdt)) return kInvalid;
    if (strict ? slen != t.orig : (t.orig > UINT64_MAX / 8 || slen > 8 * t.orig)) return kInvalid;
    std::vector<int> perm;
    std::vector<uint32_t> op_flags;
    const int ch = recognise(c, perm, op_flags);
    if (ch < 0) return kInvalid;
    if (!ch) return kUnsup;
    if (!width_ok(ch, sdt)) return kInvalid;
    const int np = ptmd_planes(ch);
    if ((int)t.planes.size() != np) return kInvalid;  // container.rs:1885-1892
    const uint64_t ratio = (uint64_t)ptmd_ratio(ch);
    if (t.orig % ratio) return kInvalid;
    const uint64_t plane_len = t.orig / ratio;
    bool all_crc = true, any_crc = false;
    // per plane: Order1ScaleAC state (offset, length, version)
    std::vector<std::array<uint64_t, 3>> st(t.planes.size(), {0, 0, 0});
    for (size_t pi = 0; pi < t.planes.size(); ++pi) {
      const PlaneRec& p = t.planes[pi];
      if (p.et_kind != 2) return p.et_kind == 1 ? kInvalid : kUnsup;
      if (p.state_source == 3) return kInvalid;  // container.rs:2104-2108
      if (!device_codec(p.codec)) return kUnsup;
      if (!p.chunked) {
        // container.rs:2051-2100: an unchunked plane's state, inline or from
        // the prelude (same version, role covered by applies_to_mask, bytes
        // matching the stored xxh64: checked whatever the codec).  Only
        // Order1ScaleAC reads it; the other codecs here ignore theirs
        // (codecs/zstd.rs:65-106 and the like).  Chunked planes carry their
        // state per frame and the record's is not read (:1975-2044).
        if (p.state_source == 1) {
          st[pi] = {p.inl_off, p.inl_len, p.state_version};
        } else if (p.state_source == 2) {
          const PreludeEnt* e = nullptr;
          for (const PreludeEnt& x : prelude)
            if (x.id == p.state_info) {
              e = &x;
              break;
            }
          if (!e || p.state_version != e->version) return kInvalid;
          if (p.role >= 1 && p.role <= 8 && !(e->mask & (1u << (p.role - 1)))) return kInvalid;
          if (xxh64_once(file + e->off, (size_t)e->len) != e->hash) return kInvalid;
          st[pi] = {e->off, e->len, e->version};
        }  // state_source 0: no state (Order1ScaleAC's decode refuses it)
        if (p.codec != kO1sac) st[pi] = {0, 0, 0};
        if (st[pi][1] > 0xFFFFFFFFull) return kInvalid;
      }
      all_crc &= p.has_crc;
      any_crc |= p.has_crc;
      if (p.chunked) {
        uint64_t tot = 0;
        for (size_t k = 0; k < p.chunks.size(); k += 2) tot += p.chunks[k + 1];
        if (tot != plane_len) return kInvalid;
        if (p.chunks.empty()) return kInvalid;
        // container.rs:1998-2009: each chunk's frame runs from its offset to
        // the next one's (the last to the payload's end), inside the payload
        for (size_t k = 0; k < p.chunks.size(); k += 2) {
          const uint64_t end = k + 2 < p.chunks.size() ? p.chunks[k + 2] : p.payload_len;
          if (p.chunks[k] > end || end > p.payload_len) return kInvalid;
        }
      }
    }
    if (any_crc && !all_crc) return kUnsup;  // the plan checks all of a tensor's planes or none
    info_flags |= all_crc ? 2u : 0u;
    out_off = (out_len + kOutAlign - 1) / kOutAlign * kOutAlign;
    out_len = out_off + t.orig;
    put(plan, out_off, 8);
    put(plan, t.orig, 8);
    put(plan, (uint64_t)ch, 1);
    put(plan, (uint64_t)np, 1);
    put(plan, (all_crc ? 1u : 0u) | (t.has_hash ? 2u : 0u), 2);
    if (t.has_hash) put(plan, t.hash, 8);
    for (int q = 0; q < np; ++q) {
      size_t j = 0;
      while (perm[j] != q) ++j;
      const PlaneRec& p = t.planes[j];
      const bool o1 = p.codec == kO1sac;
      put(plan, p.codec, 2);
      put(plan, (p.chunked ? 1u : 0u) | op_flags[(size_t)q] | (o1 ? 0x40u : 0u), 2);
      put(plan, p.chunked ? p.chunks.size() / 2 : 0, 4);
      put(plan, p.payload_off, 8);
      put(plan, p.payload_len, 8);
      put(plan, plane_len, 8);
      if (all_crc) put(plan, p.crc, 4);
      if (o1) {
        put(plan, st[j][0], 8);
        put(plan, st[j][1], 4);
        put(plan, p.row_len, 4);
        put(plan, st[j][2], 4);
      }
      for (uint32_t v : p.chunks) put(plan, v, 4);
    }
    chain_out = (uint8_t)ch;
    plan_index = (int32_t)n_plan++;
    return kOk;
  }
};

// ---- the three layouts ---------------------------------------------------

const uint8_t kMagicPtwm[9] = {0x89, 'P', 'T', 'W', 'M', '\r', '\n', 0x1a, '\n'};
const uint8_t kMagicPtwx[9] = {0x89, 'P', 'T', 'W', 'X', '\r', '\n', 0x1a, '\n'};
const uint8_t kMagicPtwc[9] = {0x89, 'P', 'T', 'W', 'C', '\r', '\n', 0x1a, '\n'};
const uint8_t kMagicPtws[5] = {0x89, 'P', 'T', 'W', 'S'};
const uint8_t kEofSentinel[8] = {0x89, 'T', 'W', 'M', 'E', 'O', 'F', 0x1a};

// legacy tensor record (tensor_record.rs:265-420)
void read_legacy_record(const uint8_t* f, uint64_t off, uint64_t len, const std::vector<Chain>& reg,
                        const std::vector<uint16_t>& reg_ids, const std::vector<EtEntry>& et, TensorRec& t) {
  Rd r(f + off, (size_t)len);
  t.rec_off = off;
  t.rec_len = len;
  const uint16_t chain_ref = r.u16();
  t.dtype = r.u16();
  t.input_format = r.u8();
  const uint8_t np = r.u8();
  const uint8_t flags = r.u8();
  r.u8();
  t.orig = r.u64();
  const uint16_t nl = r.u16();
  t.name_off = off + r.o;
  const uint8_t* name = r.take(nl);
  t.name_len = name ? nl : 0;  // a name past the record's end is not reported
  if (name && !valid_utf8(name, nl)) r.ok = false;
  r.take((4 - nl % 4) % 4);
  if (flags & 4u) {
    t.has_hash = true;
    t.hash = r.u64();
  }
  if (!r.ok) {
    t.status = kInvalid;
    return;
  }
  if (chain_ref & 0x8000u) {
    std::vector<EtEntry> inl;
    if (!read_legacy_table(r, inl) || !read_legacy_chain(r, inl, t.own_chain)) {
      t.status = kInvalid;
      return;
    }
    t.chain = &t.own_chain;
  } else {
    for (size_t i = 0; i < reg.size(); ++i)
      if (reg_ids[i] == chain_ref) t.chain = &reg[i];
    if (!t.chain) {
      t.status = kInvalid;
      return;
    }
  }
  if (flags & 1u) {  // dependencies: parsed, not used by the decode (container.rs:2161-2166)
    const uint16_t dc = r.u16();
    for (uint32_t i = 0; i < dc && r.ok; ++i) {
      const uint8_t kind = r.u8();
      const uint8_t rf = r.u8();
      r.take(r.u16());
      if (rf & 1u) r.take(32);
      if (kind < 1 || kind > 4) r.ok = false;  // RefKind::from_u8
    }
  }
  if (flags & 2u) r.take(r.u32());  // metadata (CBOR)
  t.planes.resize(np);
  for (uint32_t i = 0; i < np && r.ok; ++i) read_legacy_plane(r, off, et, t.planes[i]);
  if (!r.ok) t.status = kInvalid;
}

int64_t read_legacy(const uint8_t* f, size_t n, std::vector<TensorRec>& out, std::vector<Chain>& reg,
                    std::vector<PreludeEnt>& prelude) {
  if (n < 91 + 8 || std::memcmp(f + n - 8, kEofSentinel, 8) != 0) return kInvalid;
  Rd h(f, 91);
  const bool ptwx = std::memcmp(f, kMagicPtwx, 9) == 0;
  h.take(9);
  const uint16_t flags = h.u16();
  if ((flags & 1u) != (ptwx ? 1u : 0u)) return kInvalid;
  const uint64_t et_off = h.u64(), et_len = h.u64();
  const uint8_t* et_hash = h.take(32);  // BLAKE3 of the Extension Table section
  const uint64_t ti_off = h.u64(), ti_len = h.u64(), sp_off = h.u64(), sp_len = h.u64();
  const auto in_file = [&](uint64_t o, uint64_t l) { return o <= n && l <= n - o; };
  if (!in_file(et_off, et_len) || !in_file(ti_off, ti_len) || !in_file(sp_off, sp_len)) return kInvalid;
  if (et_len) {  // container.rs:1299: a table that does not match its hash is refused
    uint8_t got[32];
    blake3_hash(f + et_off, (size_t)et_len, got);
    if (std::memcmp(got, et_hash, 32) != 0) return kInvalid;
  }
  std::vector<EtEntry> et;
  {
    Rd r(f + et_off, (size_t)et_len);
    if (!read_legacy_table(r, et) || !r.done()) return kInvalid;
  }
  // prelude, then the chain registry, inside the shared-prelude section
  Rd sp(f + sp_off, (size_t)sp_len);
  if (!read_prelude(sp, sp_off, prelude)) return kInvalid;
  const uint16_t nc = sp.u16();
  if (!sp.ok || nc > 0x8000u) return kInvalid;
  std::vector<uint16_t> reg_ids(nc);
  reg.assign(nc, Chain{});
  for (uint32_t i = 0; i < nc; ++i) {
    reg_ids[i] = sp.u16();
    if (!sp.ok || reg_ids[i] > 0x7FFFu || !read_legacy_chain(sp, et, reg[i])) return kInvalid;
  }
  // index: u64 count, (name_hash, offset, len) entries; records in file order
  Rd ix(f + ti_off, (size_t)ti_len);
  const uint64_t cnt = ix.u64();
  if (!ix.ok || cnt > ix.left() / 24) return kInvalid;
  std::vector<std::pair<uint64_t, uint64_t>> recs((size_t)cnt);
  for (uint64_t i = 0; i < cnt; ++i) {
    ix.u64();
    recs[i].first = ix.u64();
    recs[i].second = ix.u64();
    if (!in_file(recs[i].first, recs[i].second)) return kInvalid;
  }
  std::vector<size_t> order((size_t)cnt);
  for (size_t i = 0; i < order.size(); ++i) order[i] = i;
  std::sort(order.begin(), order.end(), [&](size_t a, size_t b) { return recs[a].first < recs[b].first; });
  out.resize((size_t)cnt);
  for (size_t k = 0; k < order.size(); ++k)
    read_legacy_record(f, recs[order[k]].first, recs[order[k]].second, reg, reg_ids, et, out[k]);
  return kOk;
}

// compact tensor record (tensor_record_compact.rs:497-815)
// Whether metadata bytes are the canonical shape map that a compact record
// stores as TF_SHAPE instead (metadata.rs:54-68 encode_shape_metadata: a
// CBOR map of "shape" -> array of at most 64 unsigned ints and "dtype" ->
// a UTF-8 text string, every head in its shortest form).
bool is_shape_metadata(const uint8_t* p, size_t n) {
  Rd r(p, n);
  const auto head = [&](uint8_t major, uint64_t& v) {
    const uint8_t b = r.u8();
    if (!r.ok || (b >> 5) != major) return false;
    const uint8_t ai = b & 31u;
    if (ai < 24) {
      v = ai;
      return true;
    }
    if (ai > 27) return false;
    const int bytes = 1 << (ai - 24);
    v = 0;
    for (int i = 0; i < bytes; ++i) v = (v << 8) | r.u8();
    if (!r.ok) return false;
    const uint64_t lo = ai == 24 ? 24 : (1ull << (4 << (ai - 24)));  // shortest form only
    return v >= lo;
  };
  const auto tstr = [&](const char* want) {
    uint64_t l = 0;
    if (!head(3, l) || l != std::strlen(want)) return false;
    const uint8_t* s = r.take((size_t)l);
    return r.ok && std::memcmp(s, want, (size_t)l) == 0;
  };
  uint64_t v = 0;
  if (!head(5, v) || v != 2 || !tstr("shape")) return false;
  uint64_t nd = 0;
  if (!head(4, nd) || nd > 64) return false;
  for (uint64_t i = 0; i < nd; ++i)
    if (!head(0, v)) return false;
  if (!tstr("dtype")) return false;
  uint64_t l = 0;
  if (!head(3, l) || l > r.left()) return false;
  const uint8_t* s = r.take((size_t)l);
  return r.ok && valid_utf8(s, (size_t)l) && r.done();
}

void read_compact_record(const uint8_t* f, uint64_t off, uint64_t len, const std::vector<Chain>& reg,
                         const std::vector<EtEntry>& et, TensorRec& t) {
  Rd r(f + off, (size_t)len);
  t.rec_off = off;
  t.rec_len = len;
  const auto fail = [&]() { t.status = kInvalid; };
  const uint8_t tf = r.u8();
  if (!r.ok || (tf & 0xC0u) || ((tf & 0x10u) && !(tf & 0x08u)) || ((tf & 0x20u) && (tf & 0x08u))) return fail();
  const bool inl = (tf & 0x02u) != 0;
  uint64_t chain_id = 0;
  if (!inl) {
    chain_id = r.var();
    if (!r.ok || chain_id >= reg.size()) return fail();
  }
  t.dtype = (uint16_t)r.var_max(0xFFFF);
  t.input_format = r.u8();
  t.orig = r.var();
  std::vector<uint8_t> binding;
  bool have_binding = false;
  if (tf & 0x08u) {
    const uint64_t nd = r.var_max(64);
    if (!r.ok || nd > r.left()) return fail();
    std::vector<uint64_t> shape((size_t)nd);
    for (auto& d : shape) d = r.var();
    const char* cn = canonical_name(t.dtype);
    if (tf & 0x10u) {
      const size_t l = r.var_len();
      const uint8_t* s = r.take(l);
      if (!r.ok || !valid_utf8(s, l) || (cn && std::strlen(cn) == l && std::memcmp(cn, s, l) == 0)) return fail();
    } else if (!cn) {
      return fail();
    }
    have_binding = bound_source_params(shape, t.dtype, binding);
  } else if (tf & 0x20u) {
    // tensor_record_compact.rs:563-572: raw metadata that TF_SHAPE stores
    // is not canonical
    const size_t ml = r.var_len();
    const uint8_t* mp = r.take(ml);
    if (r.ok && is_shape_metadata(mp, ml)) return fail();
  }
  if (!r.ok) return fail();
  if (tf & 0x01u) {
    t.has_hash = true;
    t.hash = r.u64();
  }
  if (inl) {
    const size_t el = r.var_len();
    const uint8_t* ep = r.take(el);
    std::vector<EtEntry> iet;
    if (!r.ok || !read_compact_table(ep, el, iet)) return fail();
    const size_t cl = r.var_len();
    Rd cr(r.take(cl), cl);
    if (!r.ok || !read_cw2(cr, false, &iet, have_binding ? &binding : nullptr, false, t.own_chain) || !cr.done())
      return fail();
    // tensor_record_compact.rs:596-616: the inline table lists transforms
    // only, in the order the chain first uses them
    std::vector<uint16_t> first_use;
    for (const Node& nd : t.own_chain.nodes)
      if (std::find(first_use.begin(), first_use.end(), nd.op) == first_use.end()) first_use.push_back(nd.op);
    if (first_use.size() != iet.size()) return fail();
    for (size_t k = 0; k < iet.size(); ++k)
      if (iet[k].kind != 1 || iet[k].id != first_use[k]) return fail();
    t.chain = &t.own_chain;
  } else {
    const Chain& rc = reg[(size_t)chain_id];
    if (!rc.nodes.empty() && rc.nodes[0].bound) {
      if (!have_binding) return fail();
      t.own_chain = rc;
      t.own_chain.nodes[0].params = binding;
      t.own_chain.nodes[0].bound = false;
      t.chain = &t.own_chain;
    } else {
      t.chain = &rc;
    }
  }
  if (tf & 0x04u) {
    const uint64_t nd = r.var_max(0xFFFF);
    if (!r.ok || nd == 0 || nd > r.left() / 3) return fail();
    for (uint64_t i = 0; i < nd && r.ok; ++i) {
      const uint8_t kind = r.u8();
      const uint8_t rf = r.u8();
      if (kind < 1 || kind > 4 || (rf & ~1u)) return fail();
      r.take((size_t)r.var_max(0xFFFF));
      if (rf & 1u) r.take(32);
    }
  }
  const uint64_t np = r.var_max(255);
  if (!r.ok || np > r.left() / 4) return fail();
  t.planes.resize((size_t)np);
  for (size_t i = 0; i < np; ++i) {
    PlaneRec& p = t.planes[i];
    const uint8_t pf = r.u8();
    if (!r.ok || (pf & 0xC0u)) return fail();
    p.state_source = (pf >> 2) & 3u;
    const uint8_t role = r.u8();
    p.role = role;
    const uint64_t cref = r.var_max(0xFFFF);
    if (!r.ok || !known_role(role) || cref >= et.size() || et[cref].kind != 2) return fail();
    p.et_kind = 2;
    p.codec = et[cref].id;
    if (pf & 0x20u) {
      const uint8_t v = r.u8();
      const uint64_t info = r.var_max(0xFFFF);
      if (v == 0 && info == 0) return fail();
      p.state_version = v;
      p.state_info = (uint16_t)info;
    }
    const size_t inl_len = p.state_source == 1 ? r.var_len() : 0;
    p.payload_len = r.var_len();
    if (pf & 0x10u) {
      const uint64_t row = r.var_max(0xFFFFFFFFull);
      if (row == 0) return fail();
      p.row_len = (uint32_t)row;
    }
    if (pf & 0x01u) {
      p.has_crc = true;
      p.crc = r.u32();
    }
    if (pf & 0x02u) {
      const uint64_t nch = r.var_max(p.payload_len);
      if (!r.ok || nch > r.left() / 2) return fail();
      p.chunked = true;
      p.chunks.resize(2 * (size_t)nch);
      for (auto& v : p.chunks) v = (uint32_t)r.var_max(0xFFFFFFFFull);
    }
    if (p.state_source == 3) {
      r.u8();
      const uint8_t rf = r.u8();
      if (rf & ~1u) return fail();
      r.take((size_t)r.var_max(0xFFFF));
      r.u8();
      if (rf & 1u) r.take(32);
    }
    p.inl_off = off + r.o;
    p.inl_len = inl_len;
    r.take(inl_len);
    if (!r.ok || p.payload_len > r.left()) return fail();
    p.payload_off = off + r.o;
    r.take((size_t)p.payload_len);
    if (!r.ok) return fail();
  }
  if (!r.done()) return fail();
}

int64_t read_ptwc(const uint8_t* f, size_t n, std::vector<TensorRec>& out, std::vector<Chain>& reg,
                  std::vector<PreludeEnt>& prelude) {
  constexpr size_t kFooter = 16;
  if (n < 9 + 2 + kFooter || std::memcmp(f + n - 8, kEofSentinel, 8) != 0) return kInvalid;
  const size_t footer = n - kFooter;
  Rd h(f, footer);
  h.take(9);
  if (h.u16() != 0) return kInvalid;
  const uint64_t et_len = h.var(), pre_len = h.var(), reg_len = h.var();
  const size_t hash_pos = h.o;
  const uint64_t meta = h.u64();
  if (!h.ok) return kInvalid;
  const size_t hdr_end = h.o;
  uint64_t et_end, pre_end, reg_end;
  if (__builtin_add_overflow((uint64_t)hdr_end, et_len, &et_end) || et_end > footer ||
      __builtin_add_overflow(et_end, pre_len, &pre_end) || pre_end > footer ||
      __builtin_add_overflow(pre_end, reg_len, &reg_end) || reg_end > footer)
    return kInvalid;
  uint64_t index_len = 0;
  for (int i = 7; i >= 0; --i) index_len = (index_len << 8) | f[footer + (size_t)i];
  if (index_len > footer) return kInvalid;
  const uint64_t index_start = footer - index_len;
  if (reg_end > index_start) return kInvalid;
  Xxh64 x;
  x.reset();
  x.update(f, hash_pos);
  x.update(f + hdr_end, (size_t)(reg_end - hdr_end));
  if (x.digest() != meta) return kInvalid;
  std::vector<EtEntry> et;
  if (!read_compact_table(f + hdr_end, (size_t)et_len, et)) return kInvalid;
  // the prelude fills its section exactly
  Rd pr(f + et_end, (size_t)pre_len);
  if (pre_len && (!read_prelude(pr, et_end, prelude, true) || !pr.done())) return kInvalid;
  // registry (ptwc.rs:193-227)
  Rd rg(f + pre_end, (size_t)reg_len);
  const uint64_t nc = rg.var_max(0x8000);
  if (!rg.ok || nc > reg_len / 6) return kInvalid;
  reg.assign((size_t)nc, Chain{});
  for (size_t i = 0; i < nc; ++i) {
    const size_t cl = rg.var_len();
    Rd cr(rg.take(cl), cl);
    if (!rg.ok || !read_cw2(cr, false, &et, nullptr, true, reg[i]) || !cr.done()) return kInvalid;
  }
  if (!rg.done()) return kInvalid;
  // index (ptwc.rs:251-298): names and record lengths in body order
  Rd ix(f + index_start, (size_t)index_len);
  const uint64_t cnt = ix.var();
  if (!ix.ok || cnt > index_len / 3) return kInvalid;
  out.resize((size_t)cnt);
  uint64_t off = reg_end;
  for (size_t i = 0; i < cnt; ++i) {
    const uint64_t nl = ix.var_max(0xFFFF);
    if (!ix.ok || nl == 0) return kInvalid;
    out[i].name_off = index_start + ix.o;
    out[i].name_len = (uint32_t)nl;
    const uint8_t* name = ix.take((size_t)nl);
    if (!ix.ok || !valid_utf8(name, (size_t)nl)) return kInvalid;
    const uint64_t rl = ix.var();
    if (!ix.ok || rl < 3 || rl > index_start - off) return kInvalid;
    out[i].rec_off = off;
    out[i].rec_len = rl;
    off += rl;
  }
  if (!ix.done() || off != index_start) return kInvalid;
  for (size_t i = 0; i < cnt; ++i)
    for (size_t k = 0; k < i; ++k)
      if (out[k].name_len == out[i].name_len &&
          std::memcmp(f + out[k].name_off, f + out[i].name_off, out[i].name_len) == 0)
        return kInvalid;  // duplicate tensor name
  for (size_t i = 0; i < cnt; ++i) read_compact_record(f, out[i].rec_off, out[i].rec_len, reg, et, out[i]);
  return kOk;
}

// The row layout a frame's planes decode with (compact.rs:479-505: the
// terminal descriptor's layout, chain/runtime.rs:359-438).  The Source emits
// Rows { last dimension } (Flat for a scalar; transforms/source.rs:145-176),
// BytePassthrough keeps its input's layout, and the bit reorders and the
// byte and nibble splits emit Flat planes that the plane ops keep.  So a
// plane of a Source-only or Source -> BytePassthrough chain has rows of the
// last dimension and every other plane this reader plans is Flat (0).
uint32_t terminal_row_len(const Chain& c) {
  if (c.nodes.empty() || c.nodes[0].op != kOpSource) return 0;
  for (size_t i = 1; i < c.nodes.size(); ++i)
    if (c.nodes[i].op != kOpBytePassthrough) return 0;
  const std::vector<uint8_t>& sp = c.nodes[0].params;
  if (sp.empty() || sp[0] == 0 || sp.size() < 1 + 4 * (size_t)sp[0]) return 0;
  uint32_t last;
  std::memcpy(&last, sp.data() + 1 + 4 * ((size_t)sp[0] - 1), 4);
  return last;  // 0: PlaneLayout::rows(0) is None, Flat
}

// PTWS frame (compact.rs:321-550): one tensor
int64_t read_ptws(const uint8_t* f, size_t n, std::vector<TensorRec>& out) {
  out.resize(1);
  TensorRec& t = out[0];
  t.rec_off = 0;
  t.rec_len = n;
  Rd r(f, n);
  r.take(5);
  const uint8_t flags = r.u8();
  if (!r.ok || (flags & 0x80u) || ((flags & 0x02u) && (flags & 0x01u))) return kInvalid;
  t.dtype = (uint16_t)r.var_max(0xFFFF);
  t.input_format = r.u8();
  uint64_t stored = 0;
  const bool has_size = (flags & 0x40u) != 0;
  if (has_size) stored = r.var();
  std::vector<uint64_t> shape;
  bool has_shape = false;
  if (flags & 0x04u) {
    has_shape = true;
    const uint64_t nd = r.var_max(64);
    if (!r.ok) return kInvalid;
    shape.resize((size_t)nd);
    for (auto& d : shape) d = r.var();
  }
  const char* cn = canonical_name(t.dtype);
  if (flags & 0x08u) {
    if (!has_shape) return kInvalid;
    const size_t l = r.var_len();
    const uint8_t* s = r.take(l);
    if (!r.ok || !valid_utf8(s, l) || (cn && std::strlen(cn) == l && std::memcmp(cn, s, l) == 0)) return kInvalid;
  } else if (has_shape && !cn) {
    return kInvalid;
  }
  bool have_derived = false;
  uint64_t derived = 0;
  if (has_shape && public_elem_size(t.dtype)) {
    unsigned __int128 v = (unsigned)public_elem_size(t.dtype);
    have_derived = true;
    for (uint64_t d : shape) {
      v *= d;
      if (v > UINT64_MAX) have_derived = false;
      if (!have_derived) break;
    }
    derived = (uint64_t)v;
  }
  if (has_size && have_derived && stored == derived) return kInvalid;
  if (has_size) t.orig = stored;
  else if (have_derived) t.orig = derived;
  else return kInvalid;
  if (flags & 0x10u) r.take(32);  // BLAKE3 of a delta reference
  if (flags & 0x01u) {
    t.has_hash = true;
    t.hash = r.u64();
  }
  if (!r.ok) return kInvalid;
  if (flags & 0x20u) {  // stored body: the raw bytes, planned as passthrough Identity
    if (flags & 0x02u) return kInvalid;
    if (r.left() != t.orig) return kInvalid;
    t.own_chain = Chain{};
    Node src{kOpSource, false, {}};
    // a one-dimensional byte Source of orig_size bytes (u8 chain dtype)
    if (t.orig > 0xFFFFFFFFull) {
      t.status = kUnsup;
      return kOk;
    }
    src.params = {1, (uint8_t)t.orig, (uint8_t)(t.orig >> 8), (uint8_t)(t.orig >> 16), (uint8_t)(t.orig >> 24), 0x06,
                  0x00};
    t.own_chain.nodes.push_back(src);
    t.own_chain.terms.push_back(Term{0, 0});
    t.chain = &t.own_chain;
    PlaneRec p;
    p.et_kind = 2;
    p.codec = 0;
    p.payload_off = r.o;
    p.payload_len = t.orig;
    t.planes.push_back(p);
    return kOk;
  }
  std::vector<uint8_t> binding;
  const bool have_binding = has_shape && bound_source_params(shape, t.dtype, binding);
  if (!read_cw2(r, true, nullptr, have_binding ? &binding : nullptr, false, t.own_chain)) return kInvalid;
  t.chain = &t.own_chain;
  // planes in terminal order: head, [state], payload_len, [crc], payload
  const size_t np = t.own_chain.terms.size();
  t.planes.resize(np);
  const uint32_t row_len = terminal_row_len(t.own_chain);
  for (size_t i = 0; i < np; ++i) {
    PlaneRec& p = t.planes[i];
    const uint64_t head = r.var();
    if (!r.ok || (head >> 2) > 0xFFFF || !known_codec(head >> 2) || (head & 3u) == 3) return kInvalid;
    p.et_kind = 2;
    p.codec = (uint16_t)(head >> 2);
    p.row_len = row_len;
    if ((head & 3u) == 1) {  // inline state: version, length-prefixed bytes
      const uint8_t v = r.u8();
      const size_t sl = r.var_len();
      p.state_source = 1;
      p.state_version = v;
      p.inl_off = r.o;
      p.inl_len = sl;
      r.take(sl);
      if (v == 0 && sl == 0) return kInvalid;
    }
    p.payload_len = r.var_len();
    if (flags & 0x02u) {
      p.has_crc = true;
      p.crc = r.u32();
    }
    if (!r.ok || p.payload_len > r.left()) return kInvalid;
    p.payload_off = r.o;
    r.take((size_t)p.payload_len);
  }
  if (!r.done()) return kInvalid;
  return kOk;
}

}  // namespace

int64_t container_plan(const uint8_t* f, size_t n, std::vector<uint8_t>& plan,
                       std::vector<ptwm_mi355x_container_tensor>& info, uint64_t& out_len) {
  if (!f && n) return kInvalid;
  std::vector<TensorRec> recs;
  std::vector<Chain> reg;
  Builder b;
  b.file = f;
  int64_t rc;
  if (n >= 9 && (std::memcmp(f, kMagicPtwm, 9) == 0 || std::memcmp(f, kMagicPtwx, 9) == 0)) {
    rc = read_legacy(f, n, recs, reg, b.prelude);
  } else if (n >= 9 && std::memcmp(f, kMagicPtwc, 9) == 0) {
    b.strict = true;
    rc = read_ptwc(f, n, recs, reg, b.prelude);
  } else if (n >= 5 && std::memcmp(f, kMagicPtws, 5) == 0) {
    b.strict = true;
    rc = read_ptws(f, n, recs);
  } else {
    return kInvalid;  // not a .ptwm container (container.rs open: bad magic)
  }
  if (rc != kOk) return rc;
  info.assign(recs.size(), ptwm_mi355x_container_tensor{});
  for (size_t i = 0; i < recs.size(); ++i) {
    TensorRec& t = recs[i];
    ptwm_mi355x_container_tensor& o = info[i];
    o.name_offset = t.name_off;
    o.name_len = t.name_len;
    o.record_offset = t.rec_off;
    o.record_len = t.rec_len;
    o.dtype_code = t.dtype;
    o.input_format = t.input_format;
    o.orig_size = t.orig;
    o.plan_index = -1;
    if (t.status != kOk) {
      o.status = t.status;
      continue;
    }
    uint8_t ch;
    uint64_t off;
    int32_t pi;
    uint32_t fl;
    o.status = b.add(t, ch, off, pi, fl);
    o.chain = ch;
    o.out_offset = off;
    o.plan_index = pi;
    o.flags = fl;
  }
  for (int k = 0; k < 4; ++k) b.plan[8 + k] = (uint8_t)(b.n_plan >> (8 * k));
  plan.swap(b.plan);
  out_len = b.out_len;
  return (int64_t)recs.size();
}

}  // namespace ptwm

extern "C" int64_t ptwm_mi355x_container_plan(const uint8_t* file, size_t file_len, uint8_t* plan, size_t plan_cap,
                                              size_t* plan_len, ptwm_mi355x_container_tensor* tensors,
                                              size_t max_tensors, size_t* n_tensors, uint64_t* out_len) {
  std::vector<uint8_t> p;
  std::vector<ptwm_mi355x_container_tensor> info;
  uint64_t ol = 0;
  int64_t rc;
  try {
    rc = ptwm::container_plan(file, file_len, p, info, ol);
  } catch (...) {
    return -6;  // host allocation failed
  }
  if (rc < 0) return rc;
  if (plan_len) *plan_len = p.size();
  if (n_tensors) *n_tensors = info.size();
  if (out_len) *out_len = ol;
  if (p.size() > plan_cap || info.size() > max_tensors || (!plan && !p.empty()) || (!tensors && !info.empty()))
    return -2;
  if (!p.empty()) std::memcpy(plan, p.data(), p.size());
  if (!info.empty()) std::memcpy(tensors, info.data(), info.size() * sizeof(info[0]));
  int64_t planned = 0;
  for (const auto& t : info) planned += t.plan_index >= 0;
  return planned;
}
