// Per-kernel HIP-event timing hook (see esa_profile.h).  Host code only.
#include "esa_profile.h"

#include <atomic>
#include <mutex>
#include <vector>

#include "../../include/esa_hip.h"

namespace esa_profile {
namespace {

struct Record {
  int kernel;
  hipEvent_t begin, end;
};

static_assert(kNumKernels == ESA_PROFILE_KERNELS, "kernel ids and the header's ESA_PROFILE_KERNELS differ");

const char* const kNames[kNumKernels] = {
    "attn_fwd", "attn_fwd_masked", "attn_bwd_dkdv", "attn_bwd_dkdv_masked", "attn_bwd_dq",
    "attn_bwd_dq_masked", "attn_prep", "edge_gather", "segment_sum", "csr_build", "graph_attn_fwd",
    "graph_attn_bwd_dq", "graph_attn_bwd_dkdv", "edge_gather_add", "mish_fwd", "mish_bwd", "layer_norm_fwd", "layer_norm_bwd", "column_sum",
    "attn_edge_lists", "attn_edge_overflow", "segment_minmax", "linear_f32",
};

std::atomic<bool> g_enabled{false};
std::mutex g_mu;
std::vector<Record> g_records;
std::vector<hipEvent_t> g_pool;

hipEvent_t take_event() {
  if (!g_pool.empty()) {
    hipEvent_t e = g_pool.back();
    g_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

}  // namespace

bool enabled() { return g_enabled.load(std::memory_order_relaxed); }

void begin(int kernel, hipStream_t st, hipEvent_t* end_out) {
  std::lock_guard<std::mutex> lock(g_mu);
  hipEvent_t b = take_event(), e = take_event();
  if (!b || !e) { *end_out = nullptr; return; }
  if (hipEventRecord(b, st) != hipSuccess) { *end_out = nullptr; return; }
  g_records.push_back({kernel, b, e});
  *end_out = e;
}

void end(hipEvent_t end_ev, hipStream_t st) { (void)hipEventRecord(end_ev, st); }

}  // namespace esa_profile

extern "C" {

int esa_profile_enable(int on) {
  esa_profile::g_enabled.store(on != 0);
  return ESA_OK;
}

int esa_profile_collect(float* total_ms, int* launches, int capacity) {
  using namespace esa_profile;
  if (!total_ms || !launches) return ESA_ERR_NULL;
  if (capacity < kNumKernels) return ESA_ERR_SHAPE;
  for (int i = 0; i < kNumKernels; ++i) { total_ms[i] = 0.f; launches[i] = 0; }
  std::lock_guard<std::mutex> lock(g_mu);
  int rc = ESA_OK;
  for (const Record& r : g_records) {
    hipError_t e = hipEventSynchronize(r.end);
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.begin, r.end);
    if (e != hipSuccess && rc == ESA_OK) rc = (int)e;
    total_ms[r.kernel] += ms;
    launches[r.kernel] += 1;
    g_pool.push_back(r.begin);
    g_pool.push_back(r.end);
  }
  g_records.clear();
  return rc;
}

const char* esa_profile_kernel_name(int kernel) {
  return (kernel >= 0 && kernel < esa_profile::kNumKernels) ? esa_profile::kNames[kernel] : "";
}

}  // extern "C"
