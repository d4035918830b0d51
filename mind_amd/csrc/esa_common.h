// Shared device helpers for the gfx950 ESA kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define DEVI __device__ __forceinline__

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Host-side launch status: first error of a sequence of launches.
#define ESA_LAUNCH_CHECK()                          \
  do {                                              \
    hipError_t e_ = hipGetLastError();              \
    if (e_ != hipSuccess) return (int)e_;           \
  } while (0)

DEVI float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
DEVI float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// D(32x32, fp32) += A(32x16, bf16) * B(16x32, bf16).  Lane l supplies
// A[l%32][8(l/32)..+7] and B[8(l/32)..+7][l%32]; it receives
// D[8(r/4) + 4(l/32) + r%4][l%32] in accumulator register r.
DEVI f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// D(16x16, fp32) += A(16x32, bf16) * B(32x16, bf16).  Lane l supplies
// A[l%16][8(l/16)..+7] and B[8(l/16)..+7][l%16]; it receives
// D[4(l/16) + r][l%16] in accumulator register r.
DEVI f32x4 mfma16k32(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// D(16x16, fp32) += A(16x16, bf16) * B(16x16, bf16).  Lane l supplies
// A[l%16][4(l/16)..+3] and B[4(l/16)..+3][l%16]; result layout as mfma16k32.
DEVI f32x4 mfma16k16(const bf16x4& a, const bf16x4& b, const f32x4& c) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c, 0,
                                                   0, 0);
}

// Segment containing token t: the s in [0, nseg) with cu[s] <= t < cu[s+1]
// (t < cu[nseg] required).  Empty segments are skipped naturally.
DEVI int seg_of(const int* __restrict__ cu, int nseg, int t) {
  int lo = 0, hi = nseg;
  while (hi - lo > 1) {
    int mid = (lo + hi) >> 1;
    if (cu[mid] <= t) lo = mid; else hi = mid;
  }
  return lo;
}

DEVI int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Raw buffer resource over `bytes` bytes at p: a load whose byte range lies
// past the end returns zeros without touching memory.
DEVI __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
