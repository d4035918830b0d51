// Optional per-kernel timing hook: while enabled, each launch made through
// ESA_TIMED is bracketed by a pair of hipEvents recorded on its stream.
// Off by default; compute entry points never synchronise either way.
#pragma once
#include <hip/hip_runtime.h>

namespace esa_profile {

enum Kernel : int {
  kAttnFwd = 0,
  kAttnFwdMasked,
  kAttnBwdDkdv,
  kAttnBwdDkdvMasked,
  kAttnBwdDq,
  kAttnBwdDqMasked,
  kAttnPrep,        // transposes, bwd row statistics, mask metadata, plans
  kEdgeGather,
  kSegmentSum,
  kCsrBuild,
  kGraphFwd,        // node-mode (CSR adjacency) attention
  kGraphDq,
  kGraphDkdv,
  kEdgeGatherAdd,   // fused edge-token projection
  kMishFwd,         // block epilogue: mish (+ residual)
  kMishBwd,
  kLayerNormFwd,    // block prologue: pre-norm
  kLayerNormBwd,
  kColumnSum,       // Linear bias gradients
  kAttnEdgeLists,   // edge-mask key lists
  kAttnEdgeOverflow,  // edge-mask walk kernels over the overflow groups
  kSegmentMinMax,     // segmented minimum / maximum with argument
  kLinearF32,         // fp32 Linear layers of the blocks
  kNumKernels
};

bool enabled();
// Returns an event pair to record around one launch (null when disabled).
void begin(int kernel, hipStream_t st, hipEvent_t* end_out);
void end(hipEvent_t end_ev, hipStream_t st);

}  // namespace esa_profile

#define ESA_TIMED(kernel_id, stream, ...)                              \
  do {                                                                 \
    hipEvent_t esa_ev_end_ = nullptr;                                  \
    if (esa_profile::enabled()) esa_profile::begin(kernel_id, stream, &esa_ev_end_); \
    __VA_ARGS__;                                                       \
    if (esa_ev_end_) esa_profile::end(esa_ev_end_, stream);            \
  } while (0)
