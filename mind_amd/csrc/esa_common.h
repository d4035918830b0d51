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

// ---- attention dropout on the softmax probabilities, as xformers'
// memory_efficient_attention(p=...) and SDPA(dropout_p=...) apply it
// (esa/mha.py:76,82): the output is (P o Z / (1 - p)) V for a keep mask Z;
// the log-sum-exp is that of the undropped scores.  Query token q keeps key
// token k in head h iff
//   half(fmix32(row(q, h) ^ col(k)), k mod 2) >= thr,
//   row(q, h) = fmix32(s0 ^ fmix32(q * heads + h)),
//   col(k)    = fmix32(s1 ^ fmix32(floor(k / 2))),
// half(x, 0) = x mod 2^16, half(x, 1) = floor(x / 2^16): the keys 2i and
// 2i + 1 share one hash and take its low and high 16 bits.  q, k are the
// global token indices of the call ([0, total_q), [0, total_k)), s0 / s1 the
// low / high 32-bit words of the 64-bit seed (s1 xor 0x9E3779B9),
// thr = round(p 2^16) capped at 2^16 - 1, and fmix32 the 32-bit finalizer of
// MurmurHash3 (A. Appleby, SMHasher, public domain); kept values are scaled
// by inv_keep = 2^16 / (2^16 - thr), the inverse of the exact keep rate.
// A counter-based hash: the mask is a pure function of (seed, h, q, k), so
// the forward and both backward passes evaluate the same mask whatever their
// tiling, and row / column keys are computed once per token.
struct DropoutCfg {
  uint32_t s0, s1, thr_hi;   // thr_hi = thr 2^16: half(x, 1) >= thr iff x >= thr_hi,
                             // half(x, 0) >= thr iff x 2^16 (mod 2^32) >= thr_hi
  float inv_keep;            // 2^16 / (2^16 - thr)
  int heads;
};

inline DropoutCfg make_dropout(float p, unsigned long long seed, int heads) {
  DropoutCfg d{};
  d.s0 = (uint32_t)seed;
  d.s1 = (uint32_t)(seed >> 32) ^ 0x9E3779B9u;
  const double t = (double)p * 65536.0 + 0.5;
  const uint32_t thr = t >= 65535.0 ? 65535u : (uint32_t)t;
  d.thr_hi = thr << 16;
  d.inv_keep = (float)(65536.0 / (65536.0 - (double)thr));
  d.heads = heads;
  return d;
}

DEVI uint32_t fmix32(uint32_t h) {
  h ^= h >> 16;
  h *= 0x85EBCA6Bu;
  h ^= h >> 13;
  h *= 0xC2B2AE35u;
  h ^= h >> 16;
  return h;
}
DEVI uint32_t drop_row(const DropoutCfg& d, int q, int head) {
  return fmix32(d.s0 ^ fmix32((uint32_t)q * (uint32_t)d.heads + (uint32_t)head));
}
DEVI uint32_t drop_col(const DropoutCfg& d, int k) { return fmix32(d.s1 ^ fmix32((uint32_t)k >> 1)); }
// The hash of a (row, col) pair; drop_half takes key k's 16 bits of it.
DEVI uint32_t drop_bits(uint32_t row, uint32_t col) { return fmix32(row ^ col); }
DEVI bool drop_half(const DropoutCfg& d, uint32_t bits, int k) { return (bits << (((k & 1) ^ 1) << 4)) >= d.thr_hi; }
DEVI bool drop_keep(const DropoutCfg& d, uint32_t row, uint32_t col, int k) {
  return drop_half(d, drop_bits(row, col), k);
}
