// hash_host.hip -- XXH64 (seed 0) of restored device buffers on host cores.
//
// The tensor payload hash of container.rs:2185-2194 and compact.rs:441-445
// (xxhash-rust 0.8.18 xxh64) is one serial chain per buffer by its
// definition: four 64-bit accumulators stepped once per 32-byte stripe.  On
// the GPU a chain runs on single lanes at about 70 cycles per stripe (the
// 64-bit multiplies are quarter rate), i.e. ~1 s per GiB, while one host core
// runs it at memory speed.  So the buffers are copied device -> pinned host
// memory in chunks by worker threads, each on its own stream with two
// chunks in flight (the copy of chunk k+1 overlaps the hashing of chunk k),
// and every worker hashes whole buffers in order; the rate is the PCIe
// device-to-host rate.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>

#include "integrity.h"
#include "runtime.h"

namespace ptwm {

hipError_t HashWorker::init() {
  if (stream) return hipSuccess;
  for (int i = 0; i < 2; ++i) {
    note_alloc();
    hipError_t e = hipHostMalloc(&pinned[i], kHashChunk, hipHostMallocDefault);
    if (e != hipSuccess) return e;
    note_alloc();
    e = hipEventCreateWithFlags(&ev[i], hipEventDisableTiming);
    if (e != hipSuccess) return e;
  }
  // default priority: mixing stream priorities is avoided on purpose
  note_alloc();
  return hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
}

namespace {

// Worker w hashes the tasks idx[0..m) in order: chunks of kHashChunk bytes,
// copy of chunk k + 1 queued before chunk k is hashed.
int64_t run_worker(int dev, HashWorker& W, hipEvent_t ready, const std::vector<HashTask>& tasks,
                   const std::vector<size_t>& idx, std::vector<uint64_t>& out) {
  if (hipSetDevice(dev) != hipSuccess) return kInternal;
  PTWM_HIP_TRY(hipStreamWaitEvent(W.stream, ready, 0));
  struct Chunk {
    size_t task;
    uint64_t off, len;
  };
  std::vector<Chunk> chunks;
  for (size_t i : idx)
    for (uint64_t o = 0; o < tasks[i].n; o += kHashChunk)
      chunks.push_back(Chunk{i, o, std::min<uint64_t>(kHashChunk, tasks[i].n - o)});
  auto issue = [&](size_t k) -> hipError_t {
    const Chunk& c = chunks[k];
    hipError_t e = hipMemcpyAsync(W.pinned[k & 1], reinterpret_cast<const void*>(tasks[c.task].src + c.off), c.len,
                                  hipMemcpyDeviceToHost, W.stream);
    if (e != hipSuccess) return e;
    return hipEventRecord(W.ev[k & 1], W.stream);
  };
  Xxh64 st;
  st.reset();
  size_t cur = SIZE_MAX;
  if (!chunks.empty()) PTWM_HIP_TRY(issue(0));
  for (size_t k = 0; k < chunks.size(); ++k) {
    PTWM_HIP_TRY(hipEventSynchronize(W.ev[k & 1]));
    if (k + 1 < chunks.size()) PTWM_HIP_TRY(issue(k + 1));
    const Chunk& c = chunks[k];
    if (c.task != cur) {
      if (cur != SIZE_MAX) out[cur] = st.digest();
      st.reset();
      cur = c.task;
    }
    st.update(static_cast<const uint8_t*>(W.pinned[k & 1]), c.len);
  }
  if (cur != SIZE_MAX) out[cur] = st.digest();
  for (size_t i : idx)
    if (tasks[i].n == 0) {
      st.reset();
      out[i] = st.digest();
    }
  return kOk;
}

}  // namespace

int64_t xxh64_buffers(DevCtx& ctx, const std::vector<HashTask>& tasks, std::vector<uint64_t>& hashes) {
  hashes.assign(tasks.size(), 0);
  if (tasks.empty()) return kOk;
  uint64_t total = 0;
  for (const HashTask& t : tasks) total += t.n;
  // workers: enough cores to outrun the PCIe copy, no more than the tasks
  const uint32_t hw = std::max(1u, std::thread::hardware_concurrency());
  const uint32_t want = total <= 4 * kHashChunk ? 1u : std::min<uint32_t>(kHashWorkers, hw);
  const uint32_t nw = (uint32_t)std::min<size_t>(want, tasks.size());
  if (ctx.hash_workers.size() < nw) ctx.hash_workers.resize(nw);
  for (uint32_t w = 0; w < nw; ++w) PTWM_HIP_TRY(ctx.hash_workers[w].init());
  if (!ctx.hash_ready) note_alloc();
  if (!ctx.hash_ready) PTWM_HIP_TRY(hipEventCreateWithFlags(&ctx.hash_ready, hipEventDisableTiming));
  // everything queued on the call's stream (the restore) precedes the copies
  PTWM_HIP_TRY(hipEventRecord(ctx.hash_ready, ctx.stream));
  // largest buffers first, each to the least loaded worker
  std::vector<size_t> order(tasks.size());
  for (size_t i = 0; i < order.size(); ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) { return tasks[a].n > tasks[b].n; });
  std::vector<std::vector<size_t>> share(nw);
  std::vector<uint64_t> load(nw, 0);
  for (size_t i : order) {
    const uint32_t w = (uint32_t)(std::min_element(load.begin(), load.end()) - load.begin());
    share[w].push_back(i);
    load[w] += tasks[i].n + 4096;  // a small per-buffer cost keeps tiny buffers spread
  }
  // each worker's buffers in their original order
  for (auto& s : share) std::sort(s.begin(), s.end());
  std::vector<int64_t> rc(nw, kOk);
  if (nw == 1) {
    rc[0] = run_worker(ctx.dev, ctx.hash_workers[0], ctx.hash_ready, tasks, share[0], hashes);
  } else {
    std::vector<std::thread> pool;
    for (uint32_t w = 0; w < nw; ++w)
      pool.emplace_back([&, w] { rc[w] = run_worker(ctx.dev, ctx.hash_workers[w], ctx.hash_ready, tasks, share[w], hashes); });
    for (std::thread& t : pool) t.join();
  }
  // the calling thread's device is unchanged: run_worker set it only when
  // run on this thread, and then to the context's own device
  for (int64_t r : rc)
    if (r != kOk) return r;
  return kOk;
}

}  // namespace ptwm
