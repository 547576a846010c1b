// fuzz_parsers.cpp -- libFuzzer target over the library's parsers of
// untrusted bytes, built for the host with AddressSanitizer and
// UndefinedBehaviorSanitizer (tests/fuzz/Makefile):
//   first byte 0: ptwm_mi355x_container_plan over the rest (legacy PTWM/PTWX,
//                 PTWC, PTWS); every plan it writes must pass parse_plan
//                 against the file and the output size it reports
//   first byte 1: parse_plan over the rest (PTMD state bytes), against
//                 fixed input and output sizes
//   first byte 2: ptwm_mi355x_container_rewrite over the rest (PTWC, PTWS,
//                 PTWM / PTWX);
//                 what it writes must rewrite to itself and open in the reader
// A crash, a sanitizer report or a violated invariant ends the run.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../include/ptwm_mi355x.h"
#include "../../ptwm_amd/csrc/plan_types.h"

extern "C" int LLVMFuzzerTestOneInput(const uint8_t* data, size_t size) {
  if (size < 1) return 0;
  const uint8_t* p = data + 1;
  const size_t n = size - 1;
  if (data[0] == 0) {
    size_t plan_len = 0, n_t = 0;
    uint64_t out_len = 0;
    int64_t rc = ptwm_mi355x_container_plan(p, n, nullptr, 0, &plan_len, nullptr, 0, &n_t, &out_len);
    if (rc < 0 && rc != -2) return 0;
    std::vector<uint8_t> plan(plan_len ? plan_len : 1);
    std::vector<ptwm_mi355x_container_tensor> ts(n_t ? n_t : 1);
    rc = ptwm_mi355x_container_plan(p, n, plan.data(), plan_len, &plan_len, ts.data(), n_t, &n_t, &out_len);
    if (rc < 0) {
      std::fprintf(stderr, "second call failed: %lld\n", (long long)rc);
      std::abort();
    }
    ptwm::Plan parsed;
    if (ptwm::parse_plan(plan.data(), plan_len, n, out_len, parsed) != ptwm::kOk) {
      std::fprintf(stderr, "the reader wrote a plan parse_plan rejects\n");
      std::abort();
    }
    if (parsed.tensors.size() != (size_t)rc) std::abort();
    for (size_t i = 0; i < n_t; ++i)
      if (ts[i].name_offset + ts[i].name_len > n || ts[i].record_offset + ts[i].record_len > n) std::abort();
  } else if (data[0] == 1) {
    ptwm::Plan parsed;
    (void)ptwm::parse_plan(p, n, 1u << 20, 1u << 30, parsed);
  } else if (data[0] == 2) {
    size_t len = 0;
    int64_t rc = ptwm_mi355x_container_rewrite(p, n, nullptr, 0, &len);
    if (rc != -2) return 0;
    std::vector<uint8_t> a(len ? len : 1), b(len ? len : 1);
    if (ptwm_mi355x_container_rewrite(p, n, a.data(), len, &len) != (int64_t)len) std::abort();
    size_t len2 = 0;
    if (ptwm_mi355x_container_rewrite(a.data(), len, b.data(), b.size(), &len2) != (int64_t)len || len2 != len ||
        a != b) {
      std::fprintf(stderr, "a rewritten file does not rewrite to itself\n");
      std::abort();
    }
    size_t plan_len = 0, n_t = 0;
    uint64_t out_len = 0;
    (void)ptwm_mi355x_container_plan(a.data(), len, nullptr, 0, &plan_len, nullptr, 0, &n_t, &out_len);
  }
  return 0;
}
