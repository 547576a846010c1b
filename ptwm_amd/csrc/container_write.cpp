// container_write.cpp -- writers of the reference's compact layouts, and a
// complete reader of them that keeps every field, so that a file can be
// re-serialised.
//
//   compact container \x89PTWC   ptwc.rs:58-298 (header, registry, index,
//                                footer), extension/compact_table.rs:120-160,
//                                tensor_record_compact.rs:1-120 (records),
//                                chain/wire_compact.rs:1-66 (CW2), prelude.rs
//   frame             \x89PTWS   compact.rs:1-80 (one tensor)
//   legacy container  \x89PTWM   container.rs:790-1060 (section order: header,
//                     \x89PTWX   Extension Table, prelude, chain registry,
//                                records, index, EOF), header.rs,
//                                extension/table.rs:144-200, chain/wire.rs:36-130,
//                                tensor_record.rs:106-240, plane_record.rs:52-110,
//                                index.rs:18-30
//
// A File is what a container holds: for a compact container its Extension
// Table entries, prelude entries, registry chains and tensor records; for a
// frame its one tensor.  write_file() serialises a File the way the
// reference's writers do: varints are minimal LEB128, a chain's leading
// (i, 0) -> (i + 1, 0) edges are its spine, a Source whose params equal the
// tensor's bound_source_params is written bound (empty params), a frame
// stores orig_size only when its shape does not give it, and the header's
// lengths and meta_xxh64, the index and the footer are computed from the
// sections.  parse_file() reads a file into a File; writing what it read
// gives the file's bytes back, which the tests check on the reference's own
// files.  New files are built from tensors and encoded planes by
// build_compact_container() (ptwm_mi355x_container_write).
//
// Plain C++ with no device code: the fuzzer and the CPU tests build it for
// the host.
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include <algorithm>

#include "../../include/ptwm_mi355x.h"
#include "blake3_host.h"
#include "dtype_codes.h"
#include "xxh64_host.h"

namespace ptwm {
namespace cw {

using Bytes = std::vector<uint8_t>;

// ---- byte writer -------------------------------------------------------------

void put_le(Bytes& o, uint64_t v, int n) {
  for (int i = 0; i < n; ++i) o.push_back((uint8_t)(v >> (8 * i)));
}
void put_var(Bytes& o, uint64_t v) {  // minimal unsigned LEB128 (varint.rs:18-30)
  while (v >= 0x80) {
    o.push_back((uint8_t)(v | 0x80));
    v >>= 7;
  }
  o.push_back((uint8_t)v);
}
void put_bytes(Bytes& o, const Bytes& b) { o.insert(o.end(), b.begin(), b.end()); }
void put_bytes(Bytes& o, const uint8_t* p, size_t n) { o.insert(o.end(), p, p + n); }

// ---- byte reader ---------------------------------------------------------------

struct In {
  const uint8_t* b;
  size_t n, o = 0;
  bool ok = true;
  In(const uint8_t* p, size_t len) : b(p), n(p ? len : 0), ok(p != nullptr || len == 0) {}
  size_t left() const { return ok ? n - o : 0; }
  const uint8_t* take(size_t k) {
    if (!ok || n - o < k) {
      ok = false;
      return nullptr;
    }
    o += k;
    return b + o - k;
  }
  Bytes bytes(size_t k) {
    const uint8_t* p = take(k);
    return p ? Bytes(p, p + k) : Bytes();
  }
  uint64_t le(int k) {
    const uint8_t* p = take((size_t)k);
    uint64_t v = 0;
    if (p)
      for (int i = k - 1; i >= 0; --i) v = (v << 8) | p[i];
    return v;
  }
  uint8_t u8() { return (uint8_t)le(1); }
  uint64_t var() {  // canonical LEB128 of at most 10 bytes
    uint64_t v = 0;
    for (int i = 0; i < 10; ++i) {
      if (!ok || o >= n) return fail();
      const uint8_t c = b[o++];
      if (i == 9 && c > 1) return fail();
      v |= (uint64_t)(c & 0x7F) << (7 * i);
      if (!(c & 0x80)) return (i > 0 && c == 0) ? fail() : v;
    }
    return fail();
  }
  uint64_t var_max(uint64_t mx) {
    const uint64_t v = var();
    return v > mx ? fail() : v;
  }
  size_t var_len() {
    const uint64_t v = var();
    return (!ok || v > left()) ? (size_t)fail() : (size_t)v;
  }
  uint64_t fail() {
    ok = false;
    return 0;
  }
  bool done() const { return ok && o == n; }
};

// ---- chains (CW2) --------------------------------------------------------------

struct Edge {
  uint32_t src = 0, src_out = 0, dst = 0, dst_in = 0;
  bool has_role = false, has_vendor = false;
  Bytes role;    // its compact role bytes
  Bytes vendor;  // 1..65535 bytes
};
struct Term {
  uint32_t node = 0, out = 0;
  Bytes role;  // compact role bytes
};
struct Chain {
  std::vector<uint64_t> op_ref;  // OpId wire id (frame) or Extension Table index (container)
  std::vector<Bytes> params;     // per node; empty for a bound Source
  std::vector<Edge> edges;
  std::vector<Term> terms;
};

constexpr uint64_t kOpSourceWire = 0;

// Role::write (types/role.rs) parsed for its length; the bytes stay as read
bool take_role(In& r) {
  const uint8_t t = r.u8();
  switch (t) {
    case 0x00: case 0x04: case 0x07: r.u8(); break;
    case 0x01: if (r.u8() == 1) r.u8(); break;
    case 0x02: case 0x05: r.u8(); r.u8(); break;
    case 0x03: case 0x08: case 0x09: break;
    case 0x06: if (r.u8() == 1) r.le(2); break;
    case 0xFF: { r.le(2); r.take((size_t)r.le(2)); break; }
    default: r.ok = false;
  }
  return r.ok;
}

// one compact role (chain/wire_compact.rs:52-66), kept as its bytes
bool take_compact_role(In& r, Bytes& out) {
  const size_t at = r.o;
  const uint8_t b = r.u8();
  if (!r.ok) return false;
  bool good = b <= 0x04 || (b >= 0x08 && b <= 0x0C) || (b >= 0x10 && b <= 0x12) || (b >= 0x18 && b <= 0x1C) ||
              (b >= 0xC0 && b <= 0xDF);
  if (b >= 0x40 && b < 0xC0) good = (b & 7u) < ((b & 0x3Fu) >> 3) + 1;
  if (b == 0xFF) good = take_role(r);
  if (!good || !r.ok) return r.ok = false;
  out.assign(r.b + at, r.b + r.o);
  return true;
}

bool read_cw2(In& r, Chain& c) {
  c = Chain{};
  const uint64_t nn = r.var(), ne = r.var(), nt = r.var();
  if (!r.ok || nn < 1 || nn > 255 || ne > 255 || nt > 255) return false;
  for (uint64_t i = 0; i < nn; ++i) {
    c.op_ref.push_back(r.var());
    c.params.push_back(r.bytes(r.var_max(255)));
  }
  const uint64_t spine = ne ? r.var_max(ne) : 0;
  for (uint64_t i = 0; i < ne; ++i) {
    Edge e;
    if (i < spine) {
      e.src = (uint32_t)i;
      e.dst = (uint32_t)i + 1;
    } else {
      e.src = (uint32_t)r.var_max(255);
      e.src_out = (uint32_t)r.var_max(255);
      e.dst = (uint32_t)r.var_max(255);
      e.dst_in = (uint32_t)r.var_max(255);
      const uint8_t tag = r.u8();
      if (!r.ok || (tag & ~3u)) return false;
      e.has_role = tag & 1u;
      e.has_vendor = tag & 2u;
      if (e.has_role && !take_compact_role(r, e.role)) return false;
      if (e.has_vendor) {
        const uint64_t vl = r.var();
        if (vl < 1 || vl > 65535) return false;
        e.vendor = r.bytes((size_t)vl);
      }
    }
    c.edges.push_back(std::move(e));
  }
  for (uint64_t i = 0; i < nt; ++i) {
    Term t;
    const uint8_t ref = r.u8();
    if (ref == 0xFF) {
      t.node = r.u8();
      t.out = r.u8();
    } else {
      t.node = ref >> 4;
      t.out = ref & 15u;
    }
    if (!take_compact_role(r, t.role)) return false;
    c.terms.push_back(std::move(t));
  }
  return r.ok;
}

bool is_spine(const Edge& e, uint32_t i) {
  return e.src == i && e.src_out == 0 && e.dst == i + 1 && e.dst_in == 0 && !e.has_role && !e.has_vendor;
}

// write_chain_compact (chain/wire_compact.rs:108-230): the longest spine
// run is left implicit; a terminal ref is one byte when node <= 14 and
// out <= 15.  `bind`: Source params equal to it are written bound (empty).
void write_cw2(const Chain& c, const Bytes* bind, Bytes& o) {
  put_var(o, c.op_ref.size());
  put_var(o, c.edges.size());
  put_var(o, c.terms.size());
  for (size_t i = 0; i < c.op_ref.size(); ++i) {
    put_var(o, c.op_ref[i]);
    const bool bound = bind && i == 0 && c.params[i] == *bind;
    put_var(o, bound ? 0 : c.params[i].size());
    if (!bound) put_bytes(o, c.params[i]);
  }
  if (!c.edges.empty()) {
    size_t spine = 0;
    while (spine < c.edges.size() && spine < 255 && is_spine(c.edges[spine], (uint32_t)spine)) ++spine;
    put_var(o, spine);
    for (size_t i = spine; i < c.edges.size(); ++i) {
      const Edge& e = c.edges[i];
      put_var(o, e.src);
      put_var(o, e.src_out);
      put_var(o, e.dst);
      put_var(o, e.dst_in);
      o.push_back((uint8_t)((e.has_role ? 1 : 0) | (e.has_vendor ? 2 : 0)));
      if (e.has_role) put_bytes(o, e.role);
      if (e.has_vendor) {
        put_var(o, e.vendor.size());
        put_bytes(o, e.vendor);
      }
    }
  }
  for (const Term& t : c.terms) {
    if (t.node <= 14 && t.out <= 15) {
      o.push_back((uint8_t)(t.node << 4 | t.out));
    } else {
      o.push_back(0xFF);
      o.push_back((uint8_t)t.node);
      o.push_back((uint8_t)t.out);
    }
    put_bytes(o, t.role);
  }
}

// ---- records --------------------------------------------------------------------

struct Plane {
  uint8_t role = 0;
  uint64_t codec = 0;        // compact container: Extension Table index; frame: CodecId wire id
  uint8_t state_source = 0;  // 0 none, 1 inline, 2 shared, 3 external (frame: head state 0/1/2)
  uint8_t state_version = 0;
  uint64_t state_info = 0;
  Bytes state;               // inline state bytes
  uint32_t row_len = 0;      // 0: Flat layout
  bool has_crc = false;
  uint32_t crc = 0;
  bool chunked = false;
  std::vector<std::pair<uint64_t, uint64_t>> chunks;  // (offset in payload, decoded size)
  Bytes external;            // external state reference fields, as stored
  Bytes payload;
};

struct Tensor {
  std::string name;
  uint16_t dtype = 0;
  uint8_t input_format = 0;
  uint64_t orig_size = 0;
  bool has_shape = false;
  std::vector<uint64_t> shape;
  bool has_dtype_name = false;
  std::string dtype_name;
  bool has_raw_meta = false;
  Bytes raw_meta;
  bool has_hash = false;
  uint64_t hash = 0;
  bool has_delta_ref = false;  // frame only
  Bytes delta_ref;
  bool inline_chain = false;
  uint64_t chain_id = 0;       // registry chain (compact container)
  Bytes inline_table;          // compact Extension Table of an inline chain
  Chain chain;                 // inline chain (frame: the chain)
  Bytes deps;                  // dependency list after its count, as stored
  uint64_t n_deps = 0;
  bool stored = false;         // frame: raw bytes body
  Bytes raw;                   // frame: the stored body
  std::vector<Plane> planes;
};

struct TableEntry {  // compact Extension Table entry
  uint8_t tag = 0;
  uint64_t id = 0;   // tags 0x01 / 0x02
  Bytes bytes;       // tag 0x03: the name; tag 0x7F: the legacy entry bytes
};

struct PreludeEntry {  // prelude.rs:5-20
  uint16_t id = 0, codec = 0;
  uint8_t version = 0, mask = 0;
  uint64_t hash = 0;
  std::string name;
  Bytes state;
};

struct File {
  int layout = 0;  // 1 compact container, 2 frame
  std::vector<TableEntry> table;
  bool has_prelude = true;  // the prelude section is written (its count may be 0)
  std::vector<PreludeEntry> prelude;
  std::vector<Chain> registry;
  std::vector<Tensor> tensors;
};

const uint8_t kMagicPtwc[9] = {0x89, 'P', 'T', 'W', 'C', '\r', '\n', 0x1A, '\n'};
const uint8_t kMagicPtws[5] = {0x89, 'P', 'T', 'W', 'S'};
const uint8_t kEof[8] = {0x89, 'T', 'W', 'M', 'E', 'O', 'F', 0x1A};

bool read_table(const uint8_t* p, size_t n, std::vector<TableEntry>& t) {
  In r(p, n);
  const uint64_t count = r.var_max(1u << 16);
  if (!r.ok || count > n / 2) return false;
  t.assign((size_t)count, TableEntry{});
  for (TableEntry& e : t) {
    e.tag = r.u8();
    if (e.tag == 0x01 || e.tag == 0x02) e.id = r.var_max(0xFFFF);
    else if (e.tag == 0x03) e.bytes = r.bytes(r.var_max(255));
    else if (e.tag == 0x7F) e.bytes = r.bytes(r.var_len());
    else return false;
    if (!r.ok) return false;
  }
  return r.done();
}
void write_table(const std::vector<TableEntry>& t, Bytes& o) {
  put_var(o, t.size());
  for (const TableEntry& e : t) {
    o.push_back(e.tag);
    if (e.tag == 0x01 || e.tag == 0x02) {
      put_var(o, e.id);
    } else {
      put_var(o, e.bytes.size());
      put_bytes(o, e.bytes);
    }
  }
}

// parse_prelude / write_prelude (prelude.rs:65-150)
bool read_prelude(const uint8_t* p, size_t n, std::vector<PreludeEntry>& out) {
  In r(p, n);
  const uint64_t count = r.le(4);
  if (!r.ok || count > n / 22) return false;
  out.assign((size_t)count, PreludeEntry{});
  for (PreludeEntry& e : out) {
    e.id = (uint16_t)r.le(2);
    e.codec = (uint16_t)r.le(2);
    e.version = r.u8();
    e.mask = r.u8();
    if (r.le(2) != 0) return false;  // reserved
    e.hash = r.le(8);
    const size_t nl = (size_t)r.le(2);
    const uint8_t* nm = r.take(nl);
    if (!r.ok) return false;
    e.name.assign(reinterpret_cast<const char*>(nm), nl);
    const uint8_t* pad = r.take((4 - nl % 4) % 4);
    for (size_t i = 0; pad && i < (4 - nl % 4) % 4; ++i)
      if (pad[i]) return false;
    e.state = r.bytes((size_t)r.le(4));
    if (!r.ok) return false;
  }
  return r.done();
}
void write_prelude(const std::vector<PreludeEntry>& pre, Bytes& o) {
  put_le(o, pre.size(), 4);
  for (const PreludeEntry& e : pre) {
    put_le(o, e.id, 2);
    put_le(o, e.codec, 2);
    o.push_back(e.version);
    o.push_back(e.mask);
    put_le(o, 0, 2);
    put_le(o, e.hash, 8);
    put_le(o, e.name.size(), 2);
    o.insert(o.end(), e.name.begin(), e.name.end());
    o.insert(o.end(), (4 - e.name.size() % 4) % 4, 0);
    put_le(o, e.state.size(), 4);
    put_bytes(o, e.state);
  }
}

// compact record (tensor_record_compact.rs:9-54)
constexpr uint8_t kTfHash = 0x01, kTfInline = 0x02, kTfDeps = 0x04, kTfShape = 0x08, kTfName = 0x10,
                  kTfRawMeta = 0x20;
constexpr uint8_t kPfCrc = 0x01, kPfChunks = 0x02, kPfRows = 0x10, kPfExtra = 0x20;

bool read_record(const uint8_t* p, size_t n, Tensor& t) {
  In r(p, n);
  const uint8_t tf = r.u8();
  if (!r.ok || (tf & 0xC0u)) return false;
  t.inline_chain = tf & kTfInline;
  if (!t.inline_chain) t.chain_id = r.var();
  t.dtype = (uint16_t)r.var_max(0xFFFF);
  t.input_format = r.u8();
  t.orig_size = r.var();
  t.has_shape = tf & kTfShape;
  if (t.has_shape) {
    t.shape.resize((size_t)r.var_max(64));
    for (auto& d : t.shape) d = r.var();
  }
  t.has_dtype_name = tf & kTfName;
  if (t.has_dtype_name) {
    const size_t l = r.var_len();
    const uint8_t* s = r.take(l);
    if (s) t.dtype_name.assign(reinterpret_cast<const char*>(s), l);
  }
  t.has_raw_meta = tf & kTfRawMeta;
  if (t.has_raw_meta) t.raw_meta = r.bytes(r.var_len());
  t.has_hash = tf & kTfHash;
  if (t.has_hash) t.hash = r.le(8);
  if (t.inline_chain) {
    t.inline_table = r.bytes(r.var_len());
    const size_t cl = r.var_len();
    In cr(r.take(cl), cl);
    if (!r.ok || !read_cw2(cr, t.chain) || !cr.done()) return false;
  }
  if (tf & kTfDeps) {
    t.n_deps = r.var_max(0xFFFF);
    if (!r.ok || t.n_deps == 0) return false;
    const size_t at = r.o;
    for (uint64_t i = 0; i < t.n_deps && r.ok; ++i) {
      r.u8();
      const uint8_t rf = r.u8();
      r.take((size_t)r.var_max(0xFFFF));
      if (rf & 1u) r.take(32);
    }
    if (!r.ok) return false;
    t.deps.assign(p + at, p + r.o);
  }
  const uint64_t np = r.var_max(255);
  if (!r.ok) return false;
  t.planes.resize((size_t)np);
  for (Plane& q : t.planes) {
    const uint8_t pf = r.u8();
    if (!r.ok || (pf & 0xC0u)) return false;
    q.state_source = (pf >> 2) & 3u;
    q.role = r.u8();
    q.codec = r.var_max(0xFFFF);
    if (pf & kPfExtra) {
      q.state_version = r.u8();
      q.state_info = r.var_max(0xFFFF);
    }
    const size_t inl = q.state_source == 1 ? r.var_len() : 0;
    const size_t pl = r.var_len();
    if (pf & kPfRows) q.row_len = (uint32_t)r.var_max(0xFFFFFFFFull);
    q.has_crc = pf & kPfCrc;
    if (q.has_crc) q.crc = (uint32_t)r.le(4);
    q.chunked = pf & kPfChunks;
    if (q.chunked) {
      q.chunks.resize((size_t)r.var_max(pl));
      for (auto& c : q.chunks) {
        c.first = r.var_max(0xFFFFFFFFull);
        c.second = r.var_max(0xFFFFFFFFull);
      }
    }
    if (q.state_source == 3) {
      const size_t at = r.o;
      r.u8();
      const uint8_t rf = r.u8();
      r.take((size_t)r.var_max(0xFFFF));
      r.u8();
      if (rf & 1u) r.take(32);
      if (!r.ok) return false;
      q.external.assign(p + at, p + r.o);
    }
    q.state = r.bytes(inl);
    q.payload = r.bytes(pl);
    if (!r.ok) return false;
  }
  return r.done();
}

void write_record(const Tensor& t, const std::vector<bool>& registry_bound, Bytes& o) {
  const uint8_t tf = (t.has_hash ? kTfHash : 0) | (t.inline_chain ? kTfInline : 0) | (t.n_deps ? kTfDeps : 0) |
                     (t.has_shape ? kTfShape : 0) | (t.has_dtype_name ? kTfName : 0) |
                     (t.has_raw_meta ? kTfRawMeta : 0);
  o.push_back(tf);
  if (!t.inline_chain) put_var(o, t.chain_id);
  put_var(o, t.dtype);
  o.push_back(t.input_format);
  put_var(o, t.orig_size);
  if (t.has_shape) {
    put_var(o, t.shape.size());
    for (uint64_t d : t.shape) put_var(o, d);
  }
  if (t.has_dtype_name) {
    put_var(o, t.dtype_name.size());
    o.insert(o.end(), t.dtype_name.begin(), t.dtype_name.end());
  }
  if (t.has_raw_meta) {
    put_var(o, t.raw_meta.size());
    put_bytes(o, t.raw_meta);
  }
  if (t.has_hash) put_le(o, t.hash, 8);
  if (t.inline_chain) {
    put_var(o, t.inline_table.size());
    put_bytes(o, t.inline_table);
    Bytes bind, cb;
    const bool can_bind = t.has_shape && bound_source_params(t.shape, t.dtype, bind);
    write_cw2(t.chain, can_bind ? &bind : nullptr, cb);
    put_var(o, cb.size());
    put_bytes(o, cb);
  }
  (void)registry_bound;
  if (t.n_deps) {
    put_var(o, t.n_deps);
    put_bytes(o, t.deps);
  }
  put_var(o, t.planes.size());
  for (const Plane& q : t.planes) {
    const bool extra = q.state_version != 0 || q.state_info != 0;
    o.push_back((uint8_t)((q.has_crc ? kPfCrc : 0) | (q.chunked ? kPfChunks : 0) | (q.state_source << 2) |
                          (q.row_len ? kPfRows : 0) | (extra ? kPfExtra : 0)));
    o.push_back(q.role);
    put_var(o, q.codec);
    if (extra) {
      o.push_back(q.state_version);
      put_var(o, q.state_info);
    }
    if (q.state_source == 1) put_var(o, q.state.size());
    put_var(o, q.payload.size());
    if (q.row_len) put_var(o, q.row_len);
    if (q.has_crc) put_le(o, q.crc, 4);
    if (q.chunked) {
      put_var(o, q.chunks.size());
      for (const auto& c : q.chunks) {
        put_var(o, c.first);
        put_var(o, c.second);
      }
    }
    put_bytes(o, q.external);
    put_bytes(o, q.state);
    put_bytes(o, q.payload);
  }
}

// ---- the compact container ---------------------------------------------------------

bool parse_ptwc(const uint8_t* f, size_t n, File& m) {
  m = File{};
  m.layout = 1;
  if (n < 9 + 2 + 16 || std::memcmp(f, kMagicPtwc, 9) != 0 || std::memcmp(f + n - 8, kEof, 8) != 0) return false;
  const size_t footer = n - 16;
  In h(f, footer);
  h.take(9);
  if (h.le(2) != 0) return false;
  const uint64_t et_len = h.var(), pre_len = h.var(), reg_len = h.var();
  h.le(8);
  if (!h.ok) return false;
  const uint64_t et0 = h.o, pre0 = et0 + et_len, reg0 = pre0 + pre_len, body0 = reg0 + reg_len;
  if (et_len > footer || pre_len > footer || reg_len > footer || body0 > footer) return false;
  uint64_t index_len = 0;
  for (int i = 7; i >= 0; --i) index_len = (index_len << 8) | f[footer + (size_t)i];
  if (index_len > footer - body0) return false;
  const uint64_t index0 = footer - index_len;
  if (!read_table(f + et0, (size_t)et_len, m.table)) return false;
  m.has_prelude = pre_len > 0;
  if (pre_len && !read_prelude(f + pre0, (size_t)pre_len, m.prelude)) return false;
  In rg(f + reg0, (size_t)reg_len);
  const uint64_t nc = rg.var_max(0x8000);
  if (!rg.ok || nc > reg_len / 6) return false;
  m.registry.resize((size_t)nc);
  for (Chain& c : m.registry) {
    const size_t cl = rg.var_len();
    In cr(rg.take(cl), cl);
    if (!rg.ok || !read_cw2(cr, c) || !cr.done()) return false;
  }
  if (!rg.done()) return false;
  In ix(f + index0, (size_t)index_len);
  const uint64_t cnt = ix.var();
  if (!ix.ok || cnt > index_len / 3) return false;
  m.tensors.resize((size_t)cnt);
  uint64_t off = body0;
  for (Tensor& t : m.tensors) {
    const size_t nl = (size_t)ix.var_max(0xFFFF);
    const uint8_t* nm = ix.take(nl);
    const uint64_t rl = ix.var();
    if (!ix.ok || nl == 0 || rl > index0 - off) return false;
    t.name.assign(reinterpret_cast<const char*>(nm), nl);
    if (!read_record(f + off, (size_t)rl, t)) return false;
    off += rl;
  }
  return ix.done() && off == index0;
}

void write_ptwc(const File& m, Bytes& out) {
  Bytes et, pre, reg, body, index;
  write_table(m.table, et);
  if (m.has_prelude) write_prelude(m.prelude, pre);
  put_var(reg, m.registry.size());
  std::vector<bool> bound;
  for (const Chain& c : m.registry) {
    Bytes cb;
    write_cw2(c, nullptr, cb);  // a registry Source is bound when its params are empty
    put_var(reg, cb.size());
    put_bytes(reg, cb);
    bound.push_back(!c.params.empty() && c.params[0].empty());
  }
  put_var(index, m.tensors.size());
  for (const Tensor& t : m.tensors) {
    const size_t at = body.size();
    write_record(t, bound, body);
    put_var(index, t.name.size());
    index.insert(index.end(), t.name.begin(), t.name.end());
    put_var(index, body.size() - at);
  }
  // header (ptwc.rs:77-93): magic, hflags, section lengths, meta_xxh64
  out.assign(kMagicPtwc, kMagicPtwc + 9);
  put_le(out, 0, 2);
  put_var(out, et.size());
  put_var(out, pre.size());
  put_var(out, reg.size());
  Xxh64 x;
  x.reset();
  x.update(out.data(), out.size());
  x.update(et.data(), et.size());
  x.update(pre.data(), pre.size());
  x.update(reg.data(), reg.size());
  put_le(out, x.digest(), 8);
  put_bytes(out, et);
  put_bytes(out, pre);
  put_bytes(out, reg);
  put_bytes(out, body);
  put_bytes(out, index);
  put_le(out, index.size(), 8);  // footer (ptwc.rs:300-306)
  put_bytes(out, kEof, 8);
}

// ---- the frame ---------------------------------------------------------------

constexpr uint8_t kFlHash = 0x01, kFlCrc = 0x02, kFlShape = 0x04, kFlName = 0x08, kFlDelta = 0x10, kFlStored = 0x20,
                  kFlSize = 0x40;

// the raw byte count the shape gives (compact.rs size_from_shape), or false
bool size_from_shape(const std::vector<uint64_t>& shape, uint16_t dtype, uint64_t& v) {
  const int es = public_elem_size(dtype);
  if (!es) return false;
  unsigned __int128 s = (unsigned)es;
  for (uint64_t d : shape) {
    s *= d;
    if (s > UINT64_MAX) return false;
  }
  v = (uint64_t)s;
  return true;
}

bool parse_ptws(const uint8_t* f, size_t n, File& m) {
  m = File{};
  m.layout = 2;
  m.tensors.resize(1);
  Tensor& t = m.tensors[0];
  In r(f, n);
  const uint8_t* mg = r.take(5);
  if (!mg || std::memcmp(mg, kMagicPtws, 5) != 0) return false;
  const uint8_t fl = r.u8();
  if (!r.ok || (fl & 0x80u)) return false;
  t.dtype = (uint16_t)r.var_max(0xFFFF);
  t.input_format = r.u8();
  if (fl & kFlSize) t.orig_size = r.var();
  t.has_shape = fl & kFlShape;
  if (t.has_shape) {
    t.shape.resize((size_t)r.var_max(64));
    for (auto& d : t.shape) d = r.var();
  }
  t.has_dtype_name = fl & kFlName;
  if (t.has_dtype_name) {
    const size_t l = r.var_len();
    const uint8_t* s = r.take(l);
    if (s) t.dtype_name.assign(reinterpret_cast<const char*>(s), l);
  }
  t.has_delta_ref = fl & kFlDelta;
  if (t.has_delta_ref) t.delta_ref = r.bytes(32);
  t.has_hash = fl & kFlHash;
  if (t.has_hash) t.hash = r.le(8);
  if (!r.ok) return false;
  if (!(fl & kFlSize) && !(t.has_shape && size_from_shape(t.shape, t.dtype, t.orig_size))) return false;
  t.stored = fl & kFlStored;
  if (t.stored) {
    t.raw = r.bytes(r.left());
    return r.ok;
  }
  Bytes bind;
  if (!read_cw2(r, t.chain)) return false;
  if (t.has_shape && bound_source_params(t.shape, t.dtype, bind) && !t.chain.params.empty() &&
      t.chain.op_ref[0] == kOpSourceWire && t.chain.params[0].empty())
    t.chain.params[0] = bind;
  t.planes.resize(t.chain.terms.size());
  for (Plane& q : t.planes) {
    const uint64_t head = r.var();
    q.codec = head >> 2;
    q.state_source = (uint8_t)(head & 3u);
    if (q.state_source == 3) return false;
    if (q.state_source == 1) {
      q.state_version = r.u8();
      q.state = r.bytes(r.var_len());
    }
    const size_t pl = r.var_len();
    q.has_crc = fl & kFlCrc;
    if (q.has_crc) q.crc = (uint32_t)r.le(4);
    q.payload = r.bytes(pl);
    if (!r.ok) return false;
  }
  return r.done();
}

void write_ptws(const File& m, Bytes& o) {
  const Tensor& t = m.tensors[0];
  uint64_t derived = 0;
  const bool size = !(t.has_shape && size_from_shape(t.shape, t.dtype, derived) && derived == t.orig_size);
  const bool crc = !t.stored && !t.planes.empty() && t.planes[0].has_crc;
  o.assign(kMagicPtws, kMagicPtws + 5);
  o.push_back((uint8_t)((t.has_hash ? kFlHash : 0) | (crc ? kFlCrc : 0) | (t.has_shape ? kFlShape : 0) |
                        (t.has_dtype_name ? kFlName : 0) | (t.has_delta_ref ? kFlDelta : 0) |
                        (t.stored ? kFlStored : 0) | (size ? kFlSize : 0)));
  put_var(o, t.dtype);
  o.push_back(t.input_format);
  if (size) put_var(o, t.orig_size);
  if (t.has_shape) {
    put_var(o, t.shape.size());
    for (uint64_t d : t.shape) put_var(o, d);
  }
  if (t.has_dtype_name) {
    put_var(o, t.dtype_name.size());
    o.insert(o.end(), t.dtype_name.begin(), t.dtype_name.end());
  }
  if (t.has_delta_ref) put_bytes(o, t.delta_ref);
  if (t.has_hash) put_le(o, t.hash, 8);
  if (t.stored) {
    put_bytes(o, t.raw);
    return;
  }
  Bytes bind;
  const bool can_bind = t.has_shape && bound_source_params(t.shape, t.dtype, bind);
  write_cw2(t.chain, can_bind ? &bind : nullptr, o);
  for (const Plane& q : t.planes) {
    put_var(o, q.codec << 2 | q.state_source);
    if (q.state_source == 1) {
      o.push_back(q.state_version);
      put_var(o, q.state.size());
      put_bytes(o, q.state);
    }
    put_var(o, q.payload.size());
    if (crc) put_le(o, q.crc, 4);
    put_bytes(o, q.payload);
  }
}

// ---- new files from encoded planes ------------------------------------------------

// The Extension Table entry of this library's own plane codecs, in the
// legacy entry layout a compact table stores third-party entries in
// (extension/table.rs:167-200): canonical id (blake3 of extension/id.rs:
// 21-30 with the all-zero author key), label, kind 2 (plane codec), ABI 1,
// lifecycle 1, flavor hints FLAVOR_NATIVE, capabilities {"determinism":
// true, "hardware_class": "cuda"} as CBOR (the reference's device ABI slots
// this library fills are its *_cuda entry points), an empty PGP
// attestation, no install hint, no embedded WASM.
Bytes own_codec_entry(const uint8_t id[32], const char* label) {
  Bytes e(id, id + 32);
  const size_t ll = std::strlen(label);
  put_le(e, ll, 2);
  put_bytes(e, reinterpret_cast<const uint8_t*>(label), ll);
  put_le(e, 2, 2);  // Kind::PlaneCodec
  put_le(e, 1, 2);  // abi_version
  e.push_back(1);   // lifecycle
  e.push_back(2);   // FLAVOR_NATIVE
  static const char caps[] = "\xa2\x6b" "determinism" "\xf5\x6e" "hardware_class" "\x64" "cuda";
  put_le(e, sizeof(caps) - 1, 4);
  put_bytes(e, reinterpret_cast<const uint8_t*>(caps), sizeof(caps) - 1);
  e.push_back(1);   // ATTESTATION_PGP
  put_le(e, 0, 2);  // no signature bytes
  put_le(e, 0, 2);  // no install hint
  put_le(e, 0, 8);  // embedded WASM offset / length
  put_le(e, 0, 8);
  return e;
}

const uint8_t kHuffIlvId[32] = {0xcf, 0xd8, 0xcc, 0x03, 0x48, 0x3e, 0xb4, 0xa4, 0x3c, 0xdd, 0xdb,
                                0x4b, 0x3c, 0xbf, 0x95, 0xb3, 0x2e, 0xa0, 0xf3, 0x0e, 0x17, 0xe5,
                                0xec, 0x85, 0xa0, 0xb5, 0x2d, 0xe0, 0x4e, 0x8c, 0xaf, 0x04};
const uint8_t kRansIlvId[32] = {0x96, 0x8f, 0x8b, 0xe9, 0xf0, 0x6b, 0x14, 0xb5, 0x3f, 0xcd, 0x06,
                                0x66, 0x22, 0x49, 0x3f, 0x11, 0x01, 0x95, 0x4d, 0x07, 0x4d, 0x25,
                                0xd6, 0x3e, 0x78, 0x38, 0x0f, 0xe5, 0x3e, 0x1f, 0xf1, 0xf5};
constexpr uint16_t kCodecHuffIlvWire = 0x7F01, kCodecRansIlvWire = 0x7F02;

// The production chain of each decode-plan chain id (the graphs of
// python/ptwm/preprocessing/_chains.py as the reference's files store them):
// ops after the Source, ByteSplit's params, and the terminal roles by plane
// (compact roles: MantissaByte { index, of } = 0x40 + 8 (of - 1) + index,
// ExponentByte 0x19, Nibble { kind } 0x10 + kind, Value { IntN { 8 } } 0xC7)
// and the PlaneRole of each plane record (types/plane_role.rs: Value 1,
// Exponent 3, Sign 4, Mantissa 5).
struct ChainShape {
  std::vector<uint16_t> ops;
  Bytes split_params;
  std::vector<uint8_t> roles;
  std::vector<uint8_t> plane_roles;
  int elem;  // element bytes of the Source's dtype
};
bool chain_shape(int ptmd, ChainShape& s) {
  switch (ptmd) {
    case 1: s = {{0x0010, 0x0020}, {2}, {0x48, 0x19}, {5, 3}, 2}; return true;
    case 2: s = {{0x0011, 0x0020}, {4}, {0x58, 0x59, 0x5A, 0x19}, {5, 5, 5, 3}, 4}; return true;
    case 3: s = {{0x0012, 0x0021}, {}, {0x10, 0x11}, {3, 4}, 1}; return true;
    case 4: s = {{0x0013, 0x0021}, {}, {0x10, 0x11}, {3, 4}, 1}; return true;
    case 5: s = {{0x0021}, {}, {0x10, 0x11}, {1, 1}, 1}; return true;
    case 6: s = {{0x0030}, {}, {0xC7}, {1}, 1}; return true;
    default: return false;
  }
}

// Write spec ("PTWW" v1, little endian), what ptwm_mi355x_container_write
// takes:
//   u32 magic 0x57575450 | u16 version 1 | u16 layout (1 compact container,
//   2 frame) | u32 n_tensors
//   tensor: u16 name_len | name | u16 dtype_code | u8 input_format |
//           u8 chain (decode-plan chain 1..6) | u8 ndim | u64 dim x ndim |
//           u8 flags (bit 0: xxh64 follows) | [u64 xxh64] | u8 n_planes
//     plane: u16 codec wire id (0x0000 identity, 0x0001 huffman, 0x0003
//            rans, 0x0004 zstd, 0x0007 tans, 0x7F01 huff_ilv, 0x7F02
//            rans_ilv) | u8 flags (bit 0 crc, bit 1 chunked) | [u32 crc] |
//            u64 payload offset | u64 payload length (in the payload
//            buffer) | [u32 n_chunks | n x (u32 offset, u32 size)]
struct SpecPlane {
  uint16_t codec = 0;
  bool has_crc = false, chunked = false;
  uint32_t crc = 0;
  uint64_t off = 0, len = 0;
  std::vector<std::pair<uint64_t, uint64_t>> chunks;
};
struct SpecTensor {
  std::string name;
  uint16_t dtype = 0;
  uint8_t input_format = 0, chain = 0;
  std::vector<uint64_t> shape;
  bool has_hash = false;
  uint64_t hash = 0;
  std::vector<SpecPlane> planes;
};

int64_t parse_spec(const uint8_t* p, size_t n, int& layout, std::vector<SpecTensor>& out) {
  In r(p, n);
  if (r.le(4) != 0x57575450u || r.le(2) != 1) return -1;
  layout = (int)r.le(2);
  const uint64_t nt = r.le(4);
  if (!r.ok || (layout != 1 && layout != 2) || nt > n / 8 || (layout == 2 && nt != 1)) return -1;
  out.assign((size_t)nt, SpecTensor{});
  for (SpecTensor& t : out) {
    const size_t nl = (size_t)r.le(2);
    const uint8_t* nm = r.take(nl);
    if (!r.ok) return -1;
    t.name.assign(reinterpret_cast<const char*>(nm), nl);
    t.dtype = (uint16_t)r.le(2);
    t.input_format = r.u8();
    t.chain = r.u8();
    t.shape.resize(r.u8());
    for (auto& d : t.shape) d = r.le(8);
    t.has_hash = r.u8() & 1u;
    if (t.has_hash) t.hash = r.le(8);
    t.planes.resize(r.u8());
    for (SpecPlane& q : t.planes) {
      q.codec = (uint16_t)r.le(2);
      const uint8_t fl = r.u8();
      q.has_crc = fl & 1u;
      q.chunked = fl & 2u;
      if (q.has_crc) q.crc = (uint32_t)r.le(4);
      q.off = r.le(8);
      q.len = r.le(8);
      if (q.chunked) {
        q.chunks.resize((size_t)r.le(4));
        for (auto& c : q.chunks) {
          c.first = r.le(4);
          c.second = r.le(4);
        }
      }
      if (!r.ok) return -1;
    }
  }
  return r.done() ? 0 : -1;
}

bool builtin_codec(uint16_t c) { return c == 0x0000 || c == 0x0001 || c == 0x0003 || c == 0x0004 || c == 0x0007; }

// A compact container (or a frame) holding the spec's tensors, the plane
// payloads taken from `payloads`.  Registry chains are shared: one per
// decode-plan chain used, with a bound Source, so every record stores its
// shape (TF_SHAPE) and binds it.  Extension Table: the ops of the registry
// chains in first-use order, then the built-in codecs used in codec.rs
// registry order, then this library's codecs (0x7F entries).  Returns 0 or
// -1 (bad spec: unknown chain or codec, a dtype the chain cannot take, a
// shape that does not give the tensor's bytes, a plane count other than the
// chain's, a payload outside the buffer, a duplicate or empty name), -5 for
// what the layout cannot store (a frame with chunks or this library's
// codecs).
int64_t build_file(int layout, const std::vector<SpecTensor>& spec, const uint8_t* payloads, size_t payloads_len,
                   File& m) {
  m = File{};
  m.layout = layout;
  std::vector<int> chain_of_ptmd(7, -1);
  std::vector<int> op_idx(0x100, -1);
  std::vector<int> codec_used(0x80, 0);
  bool own_used[2] = {false, false};
  for (size_t i = 0; i < spec.size(); ++i) {
    const SpecTensor& t = spec[i];
    ChainShape cs;
    if (t.name.empty() || t.name.size() > 0xFFFF || !chain_shape(t.chain, cs)) return -1;
    for (size_t k = 0; k < i; ++k)
      if (spec[k].name == t.name) return -1;
    if (public_elem_size(t.dtype) != cs.elem || chain_dtype_for_public(t.dtype) < 0) return -1;
    if (t.planes.size() != cs.roles.size()) return -1;
    for (const SpecPlane& q : t.planes) {
      if (q.off > payloads_len || q.len > payloads_len - q.off) return -1;
      if (q.codec == kCodecHuffIlvWire || q.codec == kCodecRansIlvWire) {
        if (layout == 2) return -5;
        own_used[q.codec == kCodecRansIlvWire] = true;
      } else if (builtin_codec(q.codec)) {
        codec_used[q.codec] = 1;
      } else {
        return -1;
      }
      if (q.chunked && layout == 2) return -5;
    }
  }
  // registry chains, then the table: ops first, then codecs
  std::vector<int> ptmd_order;
  for (const SpecTensor& t : spec)
    if (chain_of_ptmd[t.chain] < 0) {
      chain_of_ptmd[t.chain] = (int)ptmd_order.size();
      ptmd_order.push_back(t.chain);
    }
  auto op_ref = [&](uint16_t op) -> uint64_t {
    if (op_idx[op] < 0) {
      op_idx[op] = (int)m.table.size();
      m.table.push_back(TableEntry{0x01, op, {}});
    }
    return (uint64_t)op_idx[op];
  };
  auto make_chain = [&](int ptmd, bool wire_ops, const Bytes& source_params) {
    ChainShape cs;
    chain_shape(ptmd, cs);
    Chain c;
    c.op_ref.push_back(wire_ops ? 0 : op_ref(0x0000));
    c.params.push_back(source_params);
    for (size_t k = 0; k < cs.ops.size(); ++k) {
      c.op_ref.push_back(wire_ops ? cs.ops[k] : op_ref(cs.ops[k]));
      c.params.push_back(cs.ops[k] == 0x0020 ? cs.split_params : Bytes());
      Edge e;
      e.src = (uint32_t)k;
      e.dst = (uint32_t)k + 1;
      c.edges.push_back(e);
    }
    for (size_t k = 0; k < cs.roles.size(); ++k) {
      Term tm;
      tm.node = (uint32_t)cs.ops.size();
      tm.out = (uint32_t)k;
      tm.role = {cs.roles[k]};
      c.terms.push_back(tm);
    }
    return c;
  };
  std::vector<int> codec_ref(0x80, -1);
  int own_ref[2] = {-1, -1};
  if (layout == 1) {
    for (int ptmd : ptmd_order) m.registry.push_back(make_chain(ptmd, false, Bytes()));  // bound Source
    for (uint16_t c = 0; c < 0x80; ++c)
      if (codec_used[c]) {
        codec_ref[c] = (int)m.table.size();
        m.table.push_back(TableEntry{0x02, c, {}});
      }
    for (int k = 0; k < 2; ++k)
      if (own_used[k]) {
        own_ref[k] = (int)m.table.size();
        m.table.push_back(TableEntry{0x7F, 0,
                                     own_codec_entry(k ? kRansIlvId : kHuffIlvId,
                                                     k ? "io.ptwm.mi355x.plane_codec.rans@0.1.0"
                                                       : "io.ptwm.mi355x.plane_codec@0.1.0")});
      }
  }
  for (const SpecTensor& st : spec) {
    Tensor t;
    ChainShape cs;
    chain_shape(st.chain, cs);
    t.name = st.name;
    t.dtype = st.dtype;
    t.input_format = st.input_format;
    t.has_shape = true;
    t.shape = st.shape;
    uint64_t bytes = 0;
    if (!size_from_shape(t.shape, t.dtype, bytes)) return -1;
    t.orig_size = bytes;
    t.has_hash = st.has_hash;
    t.hash = st.hash;
    Bytes bind;
    if (!bound_source_params(t.shape, t.dtype, bind)) return -1;
    if (layout == 1) {
      t.chain_id = (uint64_t)chain_of_ptmd[st.chain];
    } else {
      t.chain = make_chain(st.chain, true, bind);
      t.has_hash = st.has_hash;
    }
    for (size_t k = 0; k < st.planes.size(); ++k) {
      const SpecPlane& sq = st.planes[k];
      Plane q;
      q.role = cs.plane_roles[k];
      q.codec = layout == 2                             ? sq.codec
                : sq.codec == kCodecHuffIlvWire         ? (uint64_t)own_ref[0]
                : sq.codec == kCodecRansIlvWire         ? (uint64_t)own_ref[1]
                                                        : (uint64_t)codec_ref[sq.codec];
      q.has_crc = sq.has_crc && !(layout == 2 && st.has_hash);
      q.crc = sq.crc;
      q.chunked = sq.chunked;
      q.chunks = sq.chunks;
      q.payload.assign(payloads + sq.off, payloads + sq.off + sq.len);
      t.planes.push_back(std::move(q));
    }
    m.tensors.push_back(std::move(t));
  }
  return 0;
}

// ---- the legacy container ------------------------------------------------------------

struct LegacyChain {  // chain/wire.rs
  std::vector<uint16_t> op;  // Extension Table index per node
  std::vector<Bytes> params;
  struct E {
    uint8_t src = 0, src_out = 0, dst = 0, dst_in = 0;
    bool has_role = false;
    Bytes role;  // Role::write bytes
    Bytes vendor;
  };
  struct T {
    uint8_t node = 0, out = 0;
    Bytes role;
  };
  std::vector<E> edges;
  std::vector<T> terms;
};

struct LegacyPlane {  // plane_record.rs
  uint8_t role = 0;
  bool has_cti = true;  // PLANE_FLAG_CODEC_TABLE_IDX (always written by the current writer)
  uint16_t codec_id = 0, cti = 0;
  uint8_t state_source = 0, state_version = 0;
  uint16_t state_info = 0;
  bool has_crc = false;
  uint32_t crc = 0;
  bool chunked = false;
  std::vector<std::pair<uint32_t, uint32_t>> chunks;
  Bytes external;  // external state fields, as stored
  uint8_t layout = 0;
  uint32_t row_len = 0;
  Bytes state, payload;
};

struct LegacyTensor {  // tensor_record.rs
  uint16_t chain_ref = 0;
  uint16_t dtype = 0;
  uint8_t input_format = 0;
  std::string name;
  uint64_t orig = 0;
  bool has_hash = false;
  uint64_t hash = 0;
  std::vector<Bytes> inline_et;  // inline chain: its table's entries
  LegacyChain inline_chain;
  bool has_deps = false;
  uint16_t n_deps = 0;
  Bytes deps;
  bool has_meta = false;
  Bytes meta;
  std::vector<LegacyPlane> planes;
};

struct LegacyFile {
  bool ptwx = false;
  uint16_t flags = 0;
  std::vector<Bytes> et;  // Extension Table entries, each in the legacy entry layout
  std::vector<PreludeEntry> prelude;
  std::vector<std::pair<uint16_t, LegacyChain>> registry;
  std::vector<LegacyTensor> tensors;  // in file (append) order
};

const uint8_t kMagicPtwm[9] = {0x89, 'P', 'T', 'W', 'M', '\r', '\n', 0x1A, '\n'};
const uint8_t kMagicPtwx[9] = {0x89, 'P', 'T', 'W', 'X', '\r', '\n', 0x1A, '\n'};
constexpr size_t kLegacyHeader = 91;

// one legacy Extension Table entry (extension/table.rs:202-260), kept as its bytes
bool take_entry(In& r, Bytes& out) {
  const size_t at = r.o;
  r.take(32);
  r.take((size_t)r.le(2));
  r.le(2);
  r.le(2);
  r.u8();
  r.u8();
  const uint64_t cl = r.le(4);
  if (cl > (1u << 20)) return r.ok = false;
  r.take((size_t)cl);
  r.u8();
  r.take((size_t)r.le(2));
  r.take((size_t)r.le(2));
  r.le(8);
  r.le(8);
  if (!r.ok) return false;
  out.assign(r.b + at, r.b + r.o);
  return true;
}
bool read_legacy_table(In& r, std::vector<Bytes>& et) {
  const uint64_t count = r.le(4);
  if (!r.ok || count > 65536u || count > r.left() / 32) return r.ok = false;
  et.assign((size_t)count, Bytes());
  for (Bytes& e : et)
    if (!take_entry(r, e)) return false;
  return true;
}
void write_legacy_table(const std::vector<Bytes>& et, Bytes& o) {
  put_le(o, et.size(), 4);
  for (const Bytes& e : et) put_bytes(o, e);
}

bool read_legacy_chain(In& r, LegacyChain& c) {
  c = LegacyChain{};
  const uint32_t nn = r.u8(), ne = r.u8(), nt = r.u8();
  const size_t nl = (size_t)r.le(2), el = (size_t)r.le(2), tl = (size_t)r.le(2);
  In rn(r.take(nl), nl), re(r.take(el), el), rt(r.take(tl), tl);
  if (!r.ok) return false;
  for (uint32_t i = 0; i < nn; ++i) {
    c.op.push_back((uint16_t)rn.le(2));
    c.params.push_back(rn.bytes(rn.u8()));
  }
  for (uint32_t i = 0; i < ne; ++i) {
    LegacyChain::E e;
    e.src = re.u8();
    e.src_out = re.u8();
    e.dst = re.u8();
    e.dst_in = re.u8();
    e.has_role = re.u8() != 0;
    if (e.has_role) {
      const size_t at = re.o;
      if (!take_role(re)) return false;
      e.role.assign(re.b + at, re.b + re.o);
    }
    e.vendor = re.bytes((size_t)re.le(2));
    c.edges.push_back(std::move(e));
  }
  for (uint32_t i = 0; i < nt; ++i) {
    LegacyChain::T t;
    t.node = rt.u8();
    t.out = rt.u8();
    const size_t at = rt.o;
    if (!take_role(rt)) return false;
    t.role.assign(rt.b + at, rt.b + rt.o);
    c.terms.push_back(std::move(t));
  }
  return rn.done() && re.done() && rt.done();
}
void write_legacy_chain(const LegacyChain& c, Bytes& o) {  // chain/wire.rs:36-130
  Bytes nb, eb, tb;
  for (size_t i = 0; i < c.op.size(); ++i) {
    put_le(nb, c.op[i], 2);
    nb.push_back((uint8_t)c.params[i].size());
    put_bytes(nb, c.params[i]);
  }
  for (const auto& e : c.edges) {
    eb.insert(eb.end(), {e.src, e.src_out, e.dst, e.dst_in, (uint8_t)(e.has_role ? 1 : 0)});
    put_bytes(eb, e.role);
    put_le(eb, e.vendor.size(), 2);
    put_bytes(eb, e.vendor);
  }
  for (const auto& t : c.terms) {
    tb.push_back(t.node);
    tb.push_back(t.out);
    put_bytes(tb, t.role);
  }
  o.insert(o.end(), {(uint8_t)c.op.size(), (uint8_t)c.edges.size(), (uint8_t)c.terms.size()});
  put_le(o, nb.size(), 2);
  put_le(o, eb.size(), 2);
  put_le(o, tb.size(), 2);
  put_bytes(o, nb);
  put_bytes(o, eb);
  put_bytes(o, tb);
}

bool read_legacy_plane(In& r, LegacyPlane& p) {
  p.role = r.u8();
  const uint8_t fl = r.u8();
  p.codec_id = (uint16_t)r.le(2);
  p.has_cti = fl & 4u;
  if (p.has_cti) p.cti = (uint16_t)r.le(2);
  p.state_source = r.u8();
  p.state_version = r.u8();
  p.state_info = (uint16_t)r.le(2);
  const size_t isl = (size_t)r.le(4);
  const uint64_t pl = r.le(8);
  if (!r.ok || (fl & ~7u)) return false;
  p.has_crc = fl & 2u;
  if (p.has_crc) p.crc = (uint32_t)r.le(4);
  p.chunked = fl & 1u;
  if (p.chunked) {
    const uint64_t nc = r.le(4);
    if (!r.ok || nc > r.left() / 8) return false;
    p.chunks.resize((size_t)nc);
    for (auto& c : p.chunks) {
      c.first = (uint32_t)r.le(4);
      c.second = (uint32_t)r.le(4);
    }
  }
  if (p.state_source == 3) {
    const size_t at = r.o;
    r.u8();
    const uint8_t rf = r.u8();
    r.take((size_t)r.le(2));
    r.u8();
    if (rf & 1u) r.take(32);
    if (!r.ok) return false;
    p.external.assign(r.b + at, r.b + r.o);
  }
  p.layout = r.u8();
  if (p.layout == 1) p.row_len = (uint32_t)r.le(4);
  else if (p.layout != 0) return false;
  p.state = r.bytes(isl);
  if (!r.ok || pl > r.left()) return false;
  p.payload = r.bytes((size_t)pl);
  return r.ok;
}
void write_legacy_plane(const LegacyPlane& p, Bytes& o) {  // plane_record.rs:52-110
  o.push_back(p.role);
  o.push_back((uint8_t)((p.chunked ? 1 : 0) | (p.has_crc ? 2 : 0) | (p.has_cti ? 4 : 0)));
  put_le(o, p.codec_id, 2);
  if (p.has_cti) put_le(o, p.cti, 2);
  o.push_back(p.state_source);
  o.push_back(p.state_version);
  put_le(o, p.state_info, 2);
  put_le(o, p.state.size(), 4);
  put_le(o, p.payload.size(), 8);
  if (p.has_crc) put_le(o, p.crc, 4);
  if (p.chunked) {
    put_le(o, p.chunks.size(), 4);
    for (const auto& c : p.chunks) {
      put_le(o, c.first, 4);
      put_le(o, c.second, 4);
    }
  }
  put_bytes(o, p.external);
  o.push_back(p.layout);
  if (p.layout == 1) put_le(o, p.row_len, 4);
  put_bytes(o, p.state);
  put_bytes(o, p.payload);
}

bool read_legacy_record(const uint8_t* p, size_t n, LegacyTensor& t) {
  In r(p, n);
  t.chain_ref = (uint16_t)r.le(2);
  t.dtype = (uint16_t)r.le(2);
  t.input_format = r.u8();
  const uint8_t np = r.u8();
  const uint8_t fl = r.u8();
  if (r.u8() != 0 || (fl & ~7u)) return false;  // reserved byte, known flags
  t.orig = r.le(8);
  const size_t nl = (size_t)r.le(2);
  const uint8_t* nm = r.take(nl);
  if (!r.ok) return false;
  t.name.assign(reinterpret_cast<const char*>(nm), nl);
  const uint8_t* pad = r.take((4 - nl % 4) % 4);
  for (size_t i = 0; pad && i < (4 - nl % 4) % 4; ++i)
    if (pad[i]) return false;
  t.has_hash = fl & 4u;
  if (t.has_hash) t.hash = r.le(8);
  if (t.chain_ref & 0x8000u) {
    if (!read_legacy_table(r, t.inline_et) || !read_legacy_chain(r, t.inline_chain)) return false;
  }
  t.has_deps = fl & 1u;
  if (t.has_deps) {
    t.n_deps = (uint16_t)r.le(2);
    const size_t at = r.o;
    for (uint32_t i = 0; i < t.n_deps && r.ok; ++i) {
      r.u8();
      const uint8_t rf = r.u8();
      r.take((size_t)r.le(2));
      if (rf & 1u) r.take(32);
    }
    if (!r.ok) return false;
    t.deps.assign(p + at, p + r.o);
  }
  t.has_meta = fl & 2u;
  if (t.has_meta) t.meta = r.bytes((size_t)r.le(4));
  t.planes.resize(np);
  for (LegacyPlane& q : t.planes)
    if (!read_legacy_plane(r, q)) return false;
  return r.done();
}
void write_legacy_record(const LegacyTensor& t, Bytes& o) {  // tensor_record.rs:119-240
  put_le(o, t.chain_ref, 2);
  put_le(o, t.dtype, 2);
  o.push_back(t.input_format);
  o.push_back((uint8_t)t.planes.size());
  o.push_back((uint8_t)((t.has_deps ? 1 : 0) | (t.has_meta ? 2 : 0) | (t.has_hash ? 4 : 0)));
  o.push_back(0);
  put_le(o, t.orig, 8);
  put_le(o, t.name.size(), 2);
  o.insert(o.end(), t.name.begin(), t.name.end());
  o.insert(o.end(), (4 - t.name.size() % 4) % 4, 0);
  if (t.has_hash) put_le(o, t.hash, 8);
  if (t.chain_ref & 0x8000u) {
    write_legacy_table(t.inline_et, o);
    write_legacy_chain(t.inline_chain, o);
  }
  if (t.has_deps) {
    put_le(o, t.n_deps, 2);
    put_bytes(o, t.deps);
  }
  if (t.has_meta) {
    put_le(o, t.meta.size(), 4);
    put_bytes(o, t.meta);
  }
  for (const LegacyPlane& q : t.planes) write_legacy_plane(q, o);
}

bool parse_legacy(const uint8_t* f, size_t n, LegacyFile& m) {
  m = LegacyFile{};
  if (n < kLegacyHeader + 8 || std::memcmp(f + n - 8, kEof, 8) != 0) return false;
  m.ptwx = std::memcmp(f, kMagicPtwx, 9) == 0;
  if (!m.ptwx && std::memcmp(f, kMagicPtwm, 9) != 0) return false;
  In h(f, kLegacyHeader);
  h.take(9);
  m.flags = (uint16_t)h.le(2);
  const uint64_t et_off = h.le(8), et_len = h.le(8);
  h.take(32);
  const uint64_t ti_off = h.le(8), ti_len = h.le(8), sp_off = h.le(8), sp_len = h.le(8);
  // the writer's section order: the table right after the header, the
  // prelude right after the table, then the records, the index and EOF
  if (!h.ok || et_off != kLegacyHeader || et_len > n || sp_off != et_off + et_len || sp_len > n - sp_off ||
      ti_off < sp_off + sp_len || ti_len > n || ti_off + ti_len + 8 != n)
    return false;
  {
    In r(f + et_off, (size_t)et_len);
    if (!read_legacy_table(r, m.et) || !r.done()) return false;
  }
  In sp(f + sp_off, (size_t)sp_len);
  {
    const size_t at = sp.o;
    const uint64_t pc = sp.le(4);
    if (!sp.ok || pc > sp.left() / 22) return false;
    for (uint64_t i = 0; i < pc && sp.ok; ++i) {  // prelude.rs: fixed fields, name, pad, state
      sp.take(16);
      const size_t nl = (size_t)sp.le(2);
      sp.take(nl + (4 - nl % 4) % 4);
      sp.take((size_t)sp.le(4));
    }
    if (!sp.ok || !read_prelude(f + sp_off + at, sp.o - at, m.prelude)) return false;
  }
  const uint64_t nc = sp.le(2);
  for (uint64_t i = 0; i < nc && sp.ok; ++i) {
    const uint16_t id = (uint16_t)sp.le(2);
    LegacyChain c;
    if (!read_legacy_chain(sp, c)) return false;
    m.registry.emplace_back(id, std::move(c));
  }
  if (!sp.done()) return false;
  In ix(f + ti_off, (size_t)ti_len);
  const uint64_t cnt = ix.le(8);
  if (!ix.ok || cnt > ix.left() / 24) return false;
  std::vector<std::pair<uint64_t, uint64_t>> recs((size_t)cnt);
  for (auto& rc : recs) {
    ix.le(8);
    rc.first = ix.le(8);
    rc.second = ix.le(8);
  }
  if (!ix.done()) return false;
  std::sort(recs.begin(), recs.end());
  uint64_t at = sp_off + sp_len;
  for (const auto& rc : recs) {  // records back to back between the prelude and the index
    if (rc.first != at || rc.second > ti_off - at) return false;
    LegacyTensor t;
    if (!read_legacy_record(f + rc.first, (size_t)rc.second, t)) return false;
    m.tensors.push_back(std::move(t));
    at += rc.second;
  }
  return at == ti_off;
}

void write_legacy(const LegacyFile& m, Bytes& out) {
  Bytes et, sp, body, index;
  write_legacy_table(m.et, et);
  write_prelude(m.prelude, sp);
  put_le(sp, m.registry.size(), 2);
  for (const auto& rc : m.registry) {
    put_le(sp, rc.first, 2);
    write_legacy_chain(rc.second, sp);
  }
  const uint64_t body0 = kLegacyHeader + et.size() + sp.size();
  std::vector<std::array<uint64_t, 3>> ent;  // (name hash, offset, length)
  for (const LegacyTensor& t : m.tensors) {
    const size_t at = body.size();
    write_legacy_record(t, body);
    Xxh64 x;
    x.reset();
    x.update(reinterpret_cast<const uint8_t*>(t.name.data()), t.name.size());
    ent.push_back({x.digest(), body0 + at, body.size() - at});
  }
  std::stable_sort(ent.begin(), ent.end(), [](const auto& a, const auto& b) { return a[0] < b[0]; });
  put_le(index, ent.size(), 8);
  for (const auto& e : ent)
    for (uint64_t v : e) put_le(index, v, 8);
  // header (header.rs): magic, flags, table offset / length / BLAKE3, index
  // offset / length, prelude offset / length (prelude and registry)
  out.assign(m.ptwx ? kMagicPtwx : kMagicPtwm, (m.ptwx ? kMagicPtwx : kMagicPtwm) + 9);
  put_le(out, m.flags, 2);
  put_le(out, kLegacyHeader, 8);
  put_le(out, et.size(), 8);
  uint8_t hash[32] = {0};
  if (!et.empty()) blake3_hash(et.data(), et.size(), hash);
  put_bytes(out, hash, 32);
  put_le(out, body0 + body.size(), 8);
  put_le(out, index.size(), 8);
  put_le(out, kLegacyHeader + et.size(), 8);
  put_le(out, sp.size(), 8);
  put_bytes(out, et);
  put_bytes(out, sp);
  put_bytes(out, body);
  put_bytes(out, index);
  put_bytes(out, kEof, 8);
}

}  // namespace cw

// Re-serialise a compact container or frame through the writer: the file is
// read into its sections and records, every field kept, and written again.
int64_t container_rewrite(const uint8_t* f, size_t n, std::vector<uint8_t>& out) {
  cw::File m;
  if (n >= 9 && std::memcmp(f, cw::kMagicPtwc, 9) == 0) {
    if (!cw::parse_ptwc(f, n, m)) return -1;
    cw::write_ptwc(m, out);
    return 0;
  }
  if (n >= 5 && std::memcmp(f, cw::kMagicPtws, 5) == 0) {
    if (!cw::parse_ptws(f, n, m)) return -1;
    cw::write_ptws(m, out);
    return 0;
  }
  if (n >= 9 && (std::memcmp(f, cw::kMagicPtwm, 9) == 0 || std::memcmp(f, cw::kMagicPtwx, 9) == 0)) {
    cw::LegacyFile lm;
    if (!cw::parse_legacy(f, n, lm)) return -1;
    cw::write_legacy(lm, out);
    return 0;
  }
  return -5;
}

}  // namespace ptwm

extern "C" int64_t ptwm_mi355x_container_rewrite(const uint8_t* file, size_t file_len, uint8_t* out, size_t out_cap,
                                                 size_t* out_len) {
  if ((file_len && !file) || !out_len) return -1;
  std::vector<uint8_t> o;
  const int64_t rc = ptwm::container_rewrite(file, file_len, o);
  if (rc < 0) return rc;
  *out_len = o.size();
  if (o.size() > out_cap || (o.size() && !out)) return -2;
  if (!o.empty()) std::memcpy(out, o.data(), o.size());
  return (int64_t)o.size();
}

extern "C" int64_t ptwm_mi355x_container_write(const uint8_t* spec, size_t spec_len, const uint8_t* payloads,
                                               size_t payloads_len, uint8_t* out, size_t out_cap,
                                               size_t* out_len) {
  using namespace ptwm::cw;
  if ((spec_len && !spec) || (payloads_len && !payloads) || !out_len) return -1;
  int layout = 0;
  std::vector<SpecTensor> st;
  if (parse_spec(spec, spec_len, layout, st) < 0) return -1;
  File m;
  const int64_t rc = build_file(layout, st, payloads, payloads_len, m);
  if (rc < 0) return rc;
  std::vector<uint8_t> o;
  o.reserve(payloads_len + 2 * spec_len + 65536);  // the payloads plus record overheads of the spec's size
  if (layout == 1) write_ptwc(m, o);
  else write_ptws(m, o);
  *out_len = o.size();
  if (o.size() > out_cap || (o.size() && !out)) return -2;
  if (!o.empty()) std::memcpy(out, o.data(), o.size());
  return (int64_t)o.size();
}
