// Internal interface of the LDS-streamed prefill kernel's grouped launch
// (w4a16_prefill.hip) for the C ABI (w4a16_capi.hip).  Not installed; the
// public ABI is include/drofell_w4a16.h.
#pragma once

#include "w4a16_internal.h"

namespace dw4 {

// Several matrices of equal K, N and group size that share x (no act-order
// permutation) in one launch of the LDS-streamed prefill kernel: the plan's
// column tiles of every matrix, each matrix writing its own output (+ its
// bias, + its residual).  Unsplit plans only (splits == 1) for more than one
// matrix.
hipError_t launch_prefill2_group(const GroupArgs& a, const PrefillPlan& plan, void* ws,
                                 hipStream_t stream);

}  // namespace dw4
