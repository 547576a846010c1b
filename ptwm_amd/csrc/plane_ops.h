// plane_ops.h -- inverse plane ops on decoded terminal planes: IntDelta,
// PredictorXor, MantissaZeroStrip (chain/dispatch.rs:96-122).  They run
// between the entropy decode (and its plane CRC) and the merge.
#pragma once

#include <vector>

#include "runtime.h"

namespace ptwm {

// One inverse plane op: src (decoded terminal plane) -> dst (the plane the
// merge reads), n bytes.  src and dst are 16-byte aligned and distinct.
struct PlaneOpJob {
  uint64_t src;
  uint64_t dst;
  uint64_t n;
  uint32_t op;     // kPlaneOp*
  uint32_t param;  // element width in bytes (deltas) or k (strip)
  uint64_t tile0;  // first 4 KiB tile of the job in its launch (set by run_plane_ops)
  uint64_t aux;    // IntDelta: first slot of the job's tile sums (set by run_plane_ops)
};
static_assert(sizeof(PlaneOpJob) == 48, "PlaneOpJob layout");

// Whether the device runs this op at this parameter (PredictorXor: element
// widths 1 and 2, whose tables fit the LDS; the others always).
bool plane_op_supported(uint32_t op, uint32_t param);

// Enqueue every job on ctx.stream: the inverse ops (decode), or with
// `forward` the ops themselves (encode).  With `refused` (forward only) the
// stream is synchronised and refused[j] is nonzero for a job whose plane the
// op refuses (MantissaZeroStrip: a byte with nonzero low k bits), in the
// caller's job order.  Reorders `jobs`.  Returns kOk, kUnsupported for an
// op plane_op_supported refuses, or kInternal.
int64_t run_plane_ops(DevCtx& ctx, std::vector<PlaneOpJob>& jobs, bool forward = false,
                      std::vector<uint32_t>* refused = nullptr);

}  // namespace ptwm
