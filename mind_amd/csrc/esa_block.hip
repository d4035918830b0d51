// Pointwise epilogues of the ESA blocks on gfx950: Mish, optionally fused
// with the MAB residual add, and its backward.
//
// Semantics: F.mish / nn.Mish as the reference applies them after fc_o
// (`out + F.mish(fc_o(out))`, esa/mha.py:87, esa/mha_flash_varlen.py:120,195)
// and between the MLP Linears (esa/mlp_utils.py:24-37), evaluated in fp32 and
// rounded once to the storage type.
//
// With w = e^x and n = w (w + 2), tanh(softplus(x)) = ((1 + w)^2 - 1) /
// ((1 + w)^2 + 1) = n / (n + 2), so
//   mish(x)  = x n / (n + 2)                                  one exp, one rcp
//   mish'(x) = tanh(sp) + x sigmoid(x) sech^2(sp)
//            = n / (n + 2) + 4 x w (1 + w) / (n + 2)^2        (1 + w)^2 = n + 1
// For x > 20, tanh(softplus(x)) = 1 - 2 e^-2x rounds to 1 in fp32: mish(x)
// = x with slope 1, which also keeps w^2 inside the fp32 range.
//
// The ops are HBM-bound streams (one fp32 exp and one reciprocal per value):
// each thread moves 16-byte chunks, kUnroll of them in flight, the chunks of
// a block contiguous; misaligned pointers take an element-wise kernel.
#include "esa_common.h"
#include "esa_profile.h"
#include "../../include/esa_hip.h"

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;
constexpr float kMishLinear = 20.f;   // above: tanh(softplus(x)) == 1 in fp32

DEVI float mish_f(float x) {
  if (x > kMishLinear) return x;
  const float w = fast_exp2(x * kLog2e);
  const float n = w * (w + 2.f);
  return x * n * __builtin_amdgcn_rcpf(n + 2.f);
}

// At x = +inf the slope is NaN, as torch's mish backward gives (inf * 0);
// x is multiplied last so that a huge negative x meets w = 0 (slope 0).
DEVI float mish_grad_f(float x) {
  if (x > kMishLinear) return x < INFINITY ? 1.f : NAN;
  const float w = fast_exp2(x * kLog2e);
  const float n = w * (w + 2.f);
  const float r = __builtin_amdgcn_rcpf(n + 2.f);
  return n * r + x * (4.f * w * (1.f + w) * (r * r));
}

template <typename T> struct Chunk;
template <> struct Chunk<float> {
  static constexpr int P = 4;
  typedef f32x4 V;
  DEVI static float get(const V& v, int i) { return v[i]; }
  DEVI static void set(V& v, int i, float x) { v[i] = x; }
};
template <> struct Chunk<bf16> {
  static constexpr int P = 8;
  typedef bf16x8 V;
  DEVI static float get(const V& v, int i) { return (float)v[i]; }
  DEVI static void set(V& v, int i, float x) { v[i] = (bf16)x; }
};

// y = mish(z) (+ r), over `chunks` 16-byte chunks.  y may alias z or r: each
// chunk is read before it is written, by the same thread.
template <typename T, bool RES>
__global__ __launch_bounds__(kThreads) void mish_fwd_kernel(const T* z, const T* r, T* y, int64_t chunks) {
  typedef Chunk<T> C;
  typedef typename C::V V;
  const int64_t c0 = (int64_t)blockIdx.x * (kUnroll * kThreads) + threadIdx.x;
  V v[kUnroll], rv[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t c = c0 + u * kThreads;
    if (c < chunks) {
      v[u] = reinterpret_cast<const V*>(z)[c];
      if (RES) rv[u] = reinterpret_cast<const V*>(r)[c];
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t c = c0 + u * kThreads;
    if (c >= chunks) break;
    V o;
#pragma unroll
    for (int i = 0; i < C::P; ++i) {
      float m = mish_f(C::get(v[u], i));
      if (RES) m += C::get(rv[u], i);
      C::set(o, i, m);
    }
    reinterpret_cast<V*>(y)[c] = o;
  }
}

// dz = g * mish'(z) over `chunks` 16-byte chunks (dz may alias z or g).
template <typename T>
__global__ __launch_bounds__(kThreads) void mish_bwd_kernel(const T* z, const T* g, T* dz, int64_t chunks) {
  typedef Chunk<T> C;
  typedef typename C::V V;
  const int64_t c0 = (int64_t)blockIdx.x * (kUnroll * kThreads) + threadIdx.x;
  V v[kUnroll], gv[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t c = c0 + u * kThreads;
    if (c < chunks) {
      v[u] = reinterpret_cast<const V*>(z)[c];
      gv[u] = reinterpret_cast<const V*>(g)[c];
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t c = c0 + u * kThreads;
    if (c >= chunks) break;
    V o;
#pragma unroll
    for (int i = 0; i < C::P; ++i) C::set(o, i, C::get(gv[u], i) * mish_grad_f(C::get(v[u], i)));
    reinterpret_cast<V*>(dz)[c] = o;
  }
}

DEVI float load_f(const float* p, int64_t i) { return p[i]; }
DEVI float load_f(const bf16* p, int64_t i) { return (float)p[i]; }

// Element-wise forms over [begin, end): the tail after the last whole chunk,
// and every element when a pointer is not 16-byte aligned.
template <typename T>
__global__ __launch_bounds__(kThreads) void mish_fwd_elems_kernel(const T* z, const T* r, T* y, int64_t begin,
                                                                   int64_t end) {
  for (int64_t i = begin + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < end; i += (int64_t)gridDim.x * kThreads) {
    float m = mish_f(load_f(z, i));
    if (r) m += load_f(r, i);
    y[i] = (T)m;
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void mish_bwd_elems_kernel(const T* z, const T* g, T* dz, int64_t begin,
                                                                   int64_t end) {
  for (int64_t i = begin + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < end; i += (int64_t)gridDim.x * kThreads)
    dz[i] = (T)(load_f(g, i) * mish_grad_f(load_f(z, i)));
}

bool aligned16(const void* p) { return p == nullptr || ((uintptr_t)p & 15) == 0; }

unsigned elem_blocks(int64_t n) { return (unsigned)std::min<int64_t>((n + kThreads - 1) / kThreads, 8192); }

// Chunked launch over the aligned prefix plus an element-wise launch over the
// rest (everything when a pointer is misaligned).  `chunk_go(chunks)` and
// `elems_go(begin, end)` launch the two forms.
template <typename T, class ChunkGo, class ElemsGo>
int launch_stream(int64_t n, bool vec_ok, ChunkGo chunk_go, ElemsGo elems_go) {
  const int64_t chunks = vec_ok ? n / Chunk<T>::P : 0;
  if (chunks > 0) {
    const int64_t blocks = (chunks + kUnroll * kThreads - 1) / (kUnroll * kThreads);
    if (blocks > INT32_MAX) return ESA_ERR_SHAPE;
    chunk_go(dim3((unsigned)blocks), chunks);
  }
  const int64_t begin = chunks * Chunk<T>::P;
  if (begin < n) elems_go(dim3(elem_blocks(n - begin)), begin, n);
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

template <typename T>
int mish_fwd_typed(const T* z, const T* r, T* y, int64_t n, hipStream_t st) {
  const bool vec_ok = aligned16(z) && aligned16(r) && aligned16(y);
  int rc = ESA_OK;
  ESA_TIMED(esa_profile::kMishFwd, st,
            rc = launch_stream<T>(
                n, vec_ok,
                [&](dim3 grid, int64_t chunks) {
                  if (r) hipLaunchKernelGGL((mish_fwd_kernel<T, true>), grid, dim3(kThreads), 0, st, z, r, y, chunks);
                  else hipLaunchKernelGGL((mish_fwd_kernel<T, false>), grid, dim3(kThreads), 0, st, z, r, y, chunks);
                },
                [&](dim3 grid, int64_t b, int64_t e) {
                  hipLaunchKernelGGL(mish_fwd_elems_kernel<T>, grid, dim3(kThreads), 0, st, z, r, y, b, e);
                }));
  return rc;
}

template <typename T>
int mish_bwd_typed(const T* z, const T* g, T* dz, int64_t n, hipStream_t st) {
  const bool vec_ok = aligned16(z) && aligned16(g) && aligned16(dz);
  int rc = ESA_OK;
  ESA_TIMED(esa_profile::kMishBwd, st,
            rc = launch_stream<T>(
                n, vec_ok,
                [&](dim3 grid, int64_t chunks) {
                  hipLaunchKernelGGL(mish_bwd_kernel<T>, grid, dim3(kThreads), 0, st, z, g, dz, chunks);
                },
                [&](dim3 grid, int64_t b, int64_t e) {
                  hipLaunchKernelGGL(mish_bwd_elems_kernel<T>, grid, dim3(kThreads), 0, st, z, g, dz, b, e);
                }));
  return rc;
}

}  // namespace

extern "C" ESA_API int esa_mish_fwd(const void* z, const void* residual, int64_t n, int dtype, void* y,
                                    void* stream) {
  if (n < 0) return ESA_ERR_SHAPE;
  if (dtype != ESA_F32 && dtype != ESA_BF16) return ESA_ERR_DTYPE;
  if (n == 0) return ESA_OK;
  if (!z || !y) return ESA_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == ESA_F32)
    return mish_fwd_typed((const float*)z, (const float*)residual, (float*)y, n, st);
  return mish_fwd_typed((const bf16*)z, (const bf16*)residual, (bf16*)y, n, st);
}

extern "C" ESA_API int esa_mish_bwd(const void* z, const void* grad, int64_t n, int dtype, void* dz, void* stream) {
  if (n < 0) return ESA_ERR_SHAPE;
  if (dtype != ESA_F32 && dtype != ESA_BF16) return ESA_ERR_DTYPE;
  if (n == 0) return ESA_OK;
  if (!z || !grad || !dz) return ESA_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == ESA_F32) return mish_bwd_typed((const float*)z, (const float*)grad, (float*)dz, n, st);
  return mish_bwd_typed((const bf16*)z, (const bf16*)grad, (bf16*)dz, n, st);
}
