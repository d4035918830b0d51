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
//
// LayerNorm (the blocks' pre-norm, nn.LayerNorm(D, eps=1e-8) at
// esa/utils/norm_layers.py:36, applied at esa/masked_layers.py:418-419 and
// 478-483): fp32 row statistics (mean, biased variance), y = (x - mean) rstd
// w + b with rstd = 1 / sqrt(var + eps).  The forward can write y in fp32 and
// a bf16 copy in the same pass (under autocast the normed rows are both the
// fp32 residual and the bf16 GEMM input); the backward takes the gradients of
// both outputs and sums them, so no cast or add kernel runs beside it.
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

// ------------------------------------------------------------------ LayerNorm
// One wave per row.  Lane l holds the row's 4-feature chunks l, l + 64, ...
// (K chunks, D <= 256 K), so a chunk step of the wave reads one contiguous
// run of the row; the statistics are wave sums (butterfly: every lane ends
// with the same bits).
constexpr int kLnMaxFeatures = 2048;
constexpr int kLnMaxBlocks = 1024;   // backward: row-strided blocks (4 waves each)

DEVI float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

DEVI f32x4 load4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
DEVI f32x4 load4(const bf16* p) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
DEVI void store4(float* p, const f32x4& v) { *reinterpret_cast<f32x4*>(p) = v; }
DEVI void store4(bf16* p, const f32x4& v) {
  *reinterpret_cast<bf16x4*>(p) = bf16x4{(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
}

template <typename TX, typename TY, int K>
__global__ __launch_bounds__(256) void ln_fwd_kernel(const TX* __restrict__ x, const float* __restrict__ w,
                                                     const float* __restrict__ b, int64_t rows, int D, float eps,
                                                     TY* __restrict__ y, bf16* __restrict__ ylp,
                                                     float* __restrict__ mean, float* __restrict__ rstd) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * D;
  f32x4 v[K];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int f = 4 * (lane + 64 * k);
    v[k] = f < D ? load4(x + base + f) : f32x4{0.f, 0.f, 0.f, 0.f};
    s += (v[k][0] + v[k][1]) + (v[k][2] + v[k][3]);
  }
  const float mu = wave_sum(s) / (float)D;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    if (4 * (lane + 64 * k) < D) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = v[k][e] - mu;
        q = fmaf(d, d, q);
      }
    }
  }
  const float rs = rsqrtf(wave_sum(q) / (float)D + eps);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int f = 4 * (lane + 64 * k);
    if (f >= D) break;
    const f32x4 wv = w ? load4(w + f) : f32x4{1.f, 1.f, 1.f, 1.f};
    const f32x4 bv = b ? load4(b + f) : f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = fmaf((v[k][e] - mu) * rs, wv[e], bv[e]);
    if (y) store4(y + base + f, o);
    if (ylp) store4(ylp + base + f, o);
  }
  if (lane == 0) {
    mean[row] = mu;
    rstd[row] = rs;
  }
}

// dx = rstd (g w - mean(g w) - xhat mean(g w xhat)) + dres, g = dy + dy_lp,
// per row (dres, the gradient of x from its other uses, or none);
// dw = sum_rows g xhat, db = sum_rows g per column.  Wave w of block B takes
// rows 4 B + w, then every 4 gridDim.x further (the next row's loads are in
// flight while a row is computed); its column sums stay in registers, the
// block adds its four waves in order into part[B] (two rows of D: dw, db).
template <typename TX, typename TG, int K>
__global__ __launch_bounds__(256) void ln_bwd_kernel(const TX* __restrict__ x, const float* __restrict__ w,
                                                     const float* __restrict__ mean, const float* __restrict__ rstd,
                                                     const TG* __restrict__ dy, const bf16* __restrict__ dylp,
                                                     const TX* __restrict__ dres, int64_t rows, int D,
                                                     TX* __restrict__ dx, float* __restrict__ part) {
  __shared__ float red[4][2][256 * K];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t stride = (int64_t)gridDim.x * 4;
  f32x4 wv[K], aw[K], ab[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int f = 4 * (lane + 64 * k);
    wv[k] = (w && f < D) ? load4(w + f) : f32x4{1.f, 1.f, 1.f, 1.f};
    aw[k] = ab[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  auto load_row = [&](int64_t r, f32x4 (&xv)[K], f32x4 (&gv)[K], f32x4 (&rv)[K]) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int f = 4 * (lane + 64 * k);
      f32x4 g = f32x4{0.f, 0.f, 0.f, 0.f};
      rv[k] = g;
      if (f < D) {
        xv[k] = load4(x + r * D + f);
        if (dy) g = load4(dy + r * D + f);
        if (dylp) {
          const f32x4 h = load4(dylp + r * D + f);
#pragma unroll
          for (int e = 0; e < 4; ++e) g[e] += h[e];
        }
        if (dres) rv[k] = load4(dres + r * D + f);
      } else {
        xv[k] = g;
      }
      gv[k] = g;
    }
  };
  int64_t row = (int64_t)blockIdx.x * 4 + wave;
  f32x4 xv[K], gv[K], rv[K];
  if (row < rows) load_row(row, xv, gv, rv);
  while (row < rows) {
    const int64_t next = row + stride;
    f32x4 xn[K], gn[K], rn[K];
    if (next < rows) load_row(next, xn, gn, rn);
    const float mu = mean[row], rs = rstd[row];
    float c1 = 0.f, c2 = 0.f;
    f32x4 xh[K], dh[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xh[k][e] = (xv[k][e] - mu) * rs;
        dh[k][e] = gv[k][e] * wv[k][e];
        c1 = fmaf(dh[k][e], xh[k][e], c1);
        c2 += dh[k][e];
        aw[k][e] = fmaf(gv[k][e], xh[k][e], aw[k][e]);
        ab[k][e] += gv[k][e];
      }
    }
    c1 = wave_sum(c1) / (float)D;
    c2 = wave_sum(c2) / (float)D;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int f = 4 * (lane + 64 * k);
      if (f >= D) break;
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = rs * (dh[k][e] - c2 - xh[k][e] * c1) + rv[k][e];
      store4(dx + row * D + f, o);
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      xv[k] = xn[k];
      gv[k] = gn[k];
      rv[k] = rn[k];
    }
    row = next;
  }
  if (!part) return;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int f = 4 * (lane + 64 * k);
    if (f < D) {
      store4(&red[wave][0][f], aw[k]);
      store4(&red[wave][1][f], ab[k]);
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < D; c += 256) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
      part[((size_t)blockIdx.x * 2 + j) * D + c] = ((red[0][j][c] + red[1][j][c]) + red[2][j][c]) + red[3][j][c];
  }
}

// ---- deterministic column sums of a [nparts][width] fp32 partial matrix
// Two passes, each a fixed order: slice s of the partial rows summed per
// column into part2[s], then the slices in order; output columns below
// `split` go to out0, the rest to out1 (either may be null).  nparts = 0
// gives zeros.
constexpr int kRedSlices = 16;

__global__ __launch_bounds__(256) void col_reduce_slices_kernel(const float* __restrict__ part, int nparts, int width,
                                                                int chunk, float* __restrict__ part2) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= width) return;
  const int p0 = blockIdx.y * chunk, p1 = min(nparts, p0 + chunk);
  float a = 0.f;
#pragma unroll 8
  for (int p = p0; p < p1; ++p) a += part[(size_t)p * width + c];
  part2[(size_t)blockIdx.y * width + c] = a;
}

__global__ __launch_bounds__(256) void col_reduce_final_kernel(const float* __restrict__ part2, int slices, int width,
                                                               int split, float* __restrict__ out0,
                                                               float* __restrict__ out1) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= width) return;
  float a = 0.f;
  for (int s = 0; s < slices; ++s) a += part2[(size_t)s * width + c];
  if (c < split) {
    if (out0) out0[c] = a;
  } else if (out1) {
    out1[c - split] = a;
  }
}

size_t reduce_scratch_floats(int width) { return (size_t)kRedSlices * width; }

void reduce_columns(const float* part, int nparts, int width, float* part2, int split, float* out0, float* out1,
                    hipStream_t st) {
  const int slices = std::max(1, std::min(kRedSlices, nparts));
  const int chunk = (nparts + slices - 1) / slices;
  const unsigned cb = (unsigned)((width + 255) / 256);
  hipLaunchKernelGGL(col_reduce_slices_kernel, dim3(cb, (unsigned)slices), dim3(256), 0, st, part, nparts, width,
                     chunk, part2);
  hipLaunchKernelGGL(col_reduce_final_kernel, dim3(cb), dim3(256), 0, st, part2, slices, width, split, out0, out1);
}

// ------------------------------------------------------------------ column sums
// out[c] = sum_r x[r][c] in fp32: the bias gradient of a Linear over packed
// tokens (the autograd of the blocks' nn.Linear layers, esa/mha.py:12-15,
// esa/mlp_utils.py:18-37).  Block (i, j) sums 4-column chunks of column tile
// i over row range j, in row order, into part[j]; reduce_columns adds the
// row ranges in order.
// Row ranges: at most 1024, or 2048 from 1024 columns on, where a row range's
// blocks are few (one or two column tiles) and the extra waves keep more loads
// in flight (esa_mish_bwd_colsum at 129,850 x 2048 bf16: 404 -> 334 us; the
// column sum alone 119 -> 112 us); at 512 columns 2048 ranges gave no gain.
constexpr int kColMinRows = 32;   // rows per row range at least

int colsum_row_blocks(int64_t rows, int cols) {
  const int64_t cap = cols >= 1024 ? 2048 : 1024;
  return (int)std::max<int64_t>(1, std::min<int64_t>(cap, (rows + kColMinRows - 1) / kColMinRows));
}

template <typename T>
__global__ __launch_bounds__(256) void col_sum_partial_kernel(const T* __restrict__ x, int64_t rows, int cols,
                                                              int64_t rows_per_block, float* __restrict__ part) {
  const int c = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
  if (c >= cols) return;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per_block;
  const int64_t r1 = std::min<int64_t>(rows, r0 + rows_per_block);
  f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
  for (int64_t r = r0; r < r1; ++r) {
    const f32x4 v = load4(x + r * cols + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] += v[e];
  }
  store4(part + (size_t)blockIdx.y * cols + c, a);
}

int ln_chunks(int D) {   // K of the kernels: 4-feature chunks per lane
  const int k = (D + 255) / 256;
  return k <= 1 ? 1 : k <= 2 ? 2 : k <= 4 ? 4 : 8;
}

int ln_bwd_blocks(int64_t rows) { return (int)std::min<int64_t>(kLnMaxBlocks, (rows + 3) / 4); }

template <typename TX, typename TY>
void ln_fwd_go(int K, dim3 grid, hipStream_t st, const TX* x, const float* w, const float* b, int64_t rows, int D,
               float eps, TY* y, bf16* ylp, float* mean, float* rstd) {
#define ESA_LN_FWD(KK) hipLaunchKernelGGL((ln_fwd_kernel<TX, TY, KK>), grid, dim3(256), 0, st, x, w, b, rows, D, eps, \
                                          y, ylp, mean, rstd)
  if (K == 1) ESA_LN_FWD(1);
  else if (K == 2) ESA_LN_FWD(2);
  else if (K == 4) ESA_LN_FWD(4);
  else ESA_LN_FWD(8);
#undef ESA_LN_FWD
}

template <typename TX, typename TG>
void ln_bwd_go(int K, dim3 grid, hipStream_t st, const TX* x, const float* w, const float* mean, const float* rstd,
               const TG* dy, const bf16* dylp, const TX* dres, int64_t rows, int D, TX* dx, float* part) {
#define ESA_LN_BWD(KK) hipLaunchKernelGGL((ln_bwd_kernel<TX, TG, KK>), grid, dim3(256), 0, st, x, w, mean, rstd, dy, \
                                          dylp, dres, rows, D, dx, part)
  if (K == 1) ESA_LN_BWD(1);
  else if (K == 2) ESA_LN_BWD(2);
  else if (K == 4) ESA_LN_BWD(4);
  else ESA_LN_BWD(8);
#undef ESA_LN_BWD
}

// ------------------------------------------------------------------ MAB residual epilogue
// The block residual on top of the MAB epilogue (esa/masked_layers.py:471-472
// over esa/mha.py:87): y = x + r(o + mish(z)) with the residual stream x, y
// in fp32, z = fc_o(o) and o of type T, and r() the rounding to T that the
// MAB's own output gets.  Backward: g_o = r(g) (the gradient of o through the
// residual, and what fc_o's input gradient adds to) and dz = r(g_o mish'(z));
// x's gradient is g itself.  Four values per thread and step (16 bytes of
// fp32), kUnroll steps in flight.
DEVI float round_to(float v, float*) { return v; }
DEVI float round_to(float v, bf16*) { return (float)(bf16)v; }

template <typename T>
__global__ __launch_bounds__(kThreads) void mab_residual_fwd_kernel(const T* __restrict__ z, const T* __restrict__ o,
                                                                    const float* __restrict__ x,
                                                                    float* __restrict__ y, int64_t quads) {
  const int64_t c0 = (int64_t)blockIdx.x * (kUnroll * kThreads) + threadIdx.x;
  f32x4 zv[kUnroll], ov[kUnroll], xv[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t c = c0 + u * kThreads;
    if (c < quads) {
      zv[u] = load4(z + 4 * c);
      ov[u] = load4(o + 4 * c);
      xv[u] = load4(x + 4 * c);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t c = c0 + u * kThreads;
    if (c >= quads) break;
    f32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = xv[u][e] + round_to(ov[u][e] + mish_f(zv[u][e]), (T*)nullptr);
    store4(y + 4 * c, r);
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void mab_residual_bwd_kernel(const T* __restrict__ z,
                                                                    const float* __restrict__ g,
                                                                    T* __restrict__ dz, T* __restrict__ g_o,
                                                                    int64_t quads) {
  const int64_t c0 = (int64_t)blockIdx.x * (kUnroll * kThreads) + threadIdx.x;
  f32x4 zv[kUnroll], gv[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t c = c0 + u * kThreads;
    if (c < quads) {
      zv[u] = load4(z + 4 * c);
      gv[u] = load4(g + 4 * c);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t c = c0 + u * kThreads;
    if (c >= quads) break;
    f32x4 gl, d;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      gl[e] = round_to(gv[u][e], (T*)nullptr);
      d[e] = gl[e] * mish_grad_f(zv[u][e]);
    }
    store4(g_o + 4 * c, gl);
    store4(dz + 4 * c, d);
  }
}

// Element-wise forms over [begin, end): the tail and misaligned pointers.
template <typename T>
__global__ __launch_bounds__(kThreads) void mab_residual_fwd_elems_kernel(const T* z, const T* o, const float* x,
                                                                          float* y, int64_t begin, int64_t end) {
  for (int64_t i = begin + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < end; i += (int64_t)gridDim.x * kThreads)
    y[i] = x[i] + round_to(load_f(o, i) + mish_f(load_f(z, i)), (T*)nullptr);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void mab_residual_bwd_elems_kernel(const T* z, const float* g, T* dz, T* g_o,
                                                                          int64_t begin, int64_t end) {
  for (int64_t i = begin + (int64_t)blockIdx.x * kThreads + threadIdx.x; i < end;
       i += (int64_t)gridDim.x * kThreads) {
    const float gl = round_to(g[i], (T*)nullptr);
    g_o[i] = (T)gl;
    dz[i] = (T)(gl * mish_grad_f(load_f(z, i)));
  }
}

// Quad-chunked launch over the aligned prefix plus an element-wise launch over the rest.
template <class QuadGo, class ElemsGo>
int launch_quads(int64_t n, bool vec_ok, QuadGo quad_go, ElemsGo elems_go) {
  const int64_t quads = vec_ok ? n / 4 : 0;
  if (quads > 0) {
    const int64_t blocks = (quads + kUnroll * kThreads - 1) / (kUnroll * kThreads);
    if (blocks > INT32_MAX) return ESA_ERR_SHAPE;
    quad_go(dim3((unsigned)blocks), quads);
  }
  const int64_t begin = quads * 4;
  if (begin < n) elems_go(dim3(elem_blocks(n - begin)), begin, n);
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

template <typename T>
int mab_residual_fwd_typed(const T* z, const T* o, const float* x, float* y, int64_t n, hipStream_t st) {
  const bool vec_ok = aligned16(z) && aligned16(o) && aligned16(x) && aligned16(y);
  int rc = ESA_OK;
  ESA_TIMED(esa_profile::kMishFwd, st,
            rc = launch_quads(
                n, vec_ok,
                [&](dim3 grid, int64_t quads) {
                  hipLaunchKernelGGL(mab_residual_fwd_kernel<T>, grid, dim3(kThreads), 0, st, z, o, x, y, quads);
                },
                [&](dim3 grid, int64_t b, int64_t e) {
                  hipLaunchKernelGGL(mab_residual_fwd_elems_kernel<T>, grid, dim3(kThreads), 0, st, z, o, x, y, b,
                                     e);
                }));
  return rc;
}

template <typename T>
int mab_residual_bwd_typed(const T* z, const float* g, T* dz, T* g_o, int64_t n, hipStream_t st) {
  const bool vec_ok = aligned16(z) && aligned16(g) && aligned16(dz) && aligned16(g_o);
  int rc = ESA_OK;
  ESA_TIMED(esa_profile::kMishBwd, st,
            rc = launch_quads(
                n, vec_ok,
                [&](dim3 grid, int64_t quads) {
                  hipLaunchKernelGGL(mab_residual_bwd_kernel<T>, grid, dim3(kThreads), 0, st, z, g, dz, g_o, quads);
                },
                [&](dim3 grid, int64_t b, int64_t e) {
                  hipLaunchKernelGGL(mab_residual_bwd_elems_kernel<T>, grid, dim3(kThreads), 0, st, z, g, dz, g_o, b,
                                     e);
                }));
  return rc;
}

// Mish backward of a [rows, cols] tensor together with the column sums of
// its result, the bias gradient of the Linear whose output z is (an MLP's
// Linear -> Mish, esa/mlp_utils.py:18-37): dz = r(g mish'(z)) as
// mish_bwd_kernel computes it, and the grid, row ranges and order of
// col_sum_partial_kernel over the rounded dz, so the partials (and, through
// reduce_columns, the sums) equal esa_column_sum's over the stored dz.  One
// pass instead of a second read of dz.
// Raw 16- or 8-byte row chunk of CPT columns as the kernel loads it.
template <typename T, int CPT> struct RowChunk;
template <> struct RowChunk<float, 4> {
  typedef f32x4 V;
  DEVI static float get(const V& v, int e) { return v[e]; }
};
template <> struct RowChunk<bf16, 8> {
  typedef bf16x8 V;
  DEVI static float get(const V& v, int e) { return (float)v[e]; }
};
template <> struct RowChunk<bf16, 4> {
  typedef bf16x4 V;
  DEVI static float get(const V& v, int e) { return (float)v[e]; }
};

template <typename T, int CPT>
__global__ __launch_bounds__(256) void mish_bwd_colsum_kernel(const T* __restrict__ z, const T* __restrict__ g,
                                                              int64_t rows, int cols, int64_t rows_per_block,
                                                              T* __restrict__ dz, float* __restrict__ part) {
  // The sums add the stored (rounded) products: without this the compiler keeps a multiply for the store and
  // fuses g * mish'(z) into the accumulation (an fma of the unrounded product).  mish_grad_f keeps its own.
#pragma clang fp contract(off)
  typedef RowChunk<T, CPT> R;
  typedef typename R::V V;
  constexpr int Q = CPT / 4;   // 4-column quads per thread: one 16-byte access per row for bf16 (CPT = 8)
  constexpr int U = 4;         // rows per batch; two batches in registers
  const int c = CPT * (blockIdx.x * blockDim.x + threadIdx.x);
  if (c >= cols) return;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per_block;
  const int64_t r1 = std::min<int64_t>(rows, r0 + rows_per_block);
  f32x4 a[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) a[q] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Each thread walks its rows in order; the loads of the next batch of U
  // rows are issued before the current batch's arithmetic, so a wave keeps
  // two batches of loads in flight (the slope's range test is a branch per
  // element, which the compiler will not hoist loads across).  Loads past r1
  // re-read row r1 - 1 and are not used: the waits stay exact.
  V zr[2][U], gr[2][U];
  auto load = [&](int b, int64_t rb) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t r = std::min<int64_t>(rb + u, r1 - 1);
      zr[b][u] = *reinterpret_cast<const V*>(z + r * cols + c);
      gr[b][u] = *reinterpret_cast<const V*>(g + r * cols + c);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto batch = [&](int b, int64_t rb) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (rb + u >= r1) break;   // uniform over the block
      f32x4 d[Q];
#pragma unroll
      for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          d[q][e] = round_to(R::get(gr[b][u], 4 * q + e) * mish_grad_f(R::get(zr[b][u], 4 * q + e)), (T*)nullptr);
      T* out = dz + (rb + u) * cols + c;
      if constexpr (Q == 2) {
        bf16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (bf16)d[e / 4][e % 4];
        *reinterpret_cast<bf16x8*>(out) = o;
      } else {
        store4(out, d[0]);
      }
#pragma unroll
      for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) a[q][e] += d[q][e];
    }
  };
  if (r0 < r1) {
    load(0, r0);
    for (int64_t rb = r0; rb < r1; rb += 2 * U) {
      load(1, rb + U);
      batch(0, rb);
      if (rb + U >= r1) break;
      load(0, rb + 2 * U);
      batch(1, rb + U);
    }
  }
#pragma unroll
  for (int q = 0; q < Q; ++q) store4(part + (size_t)blockIdx.y * cols + c + 4 * q, a[q]);
}

}  // namespace

extern "C" ESA_API int esa_layer_norm_fwd(const void* x, int x_dtype, const float* weight, const float* bias,
                                          int64_t rows, int features, float eps, void* y, int y_dtype, void* y_lp,
                                          float* mean, float* rstd, void* stream) {
  if (rows < 0 || features < 4 || features > kLnMaxFeatures || features % 4) return ESA_ERR_SHAPE;
  if ((x_dtype != ESA_F32 && x_dtype != ESA_BF16) || (y && y_dtype != ESA_F32 && y_dtype != ESA_BF16))
    return ESA_ERR_DTYPE;
  if (rows == 0) return ESA_OK;
  if (!x || !mean || !rstd || (!y && !y_lp)) return ESA_ERR_NULL;
  if (!aligned16(x) || !aligned16(weight) || !aligned16(bias) || !aligned16(y) || !aligned16(y_lp))
    return ESA_ERR_ALIGN;
  if ((rows + 3) / 4 > INT32_MAX) return ESA_ERR_SHAPE;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)((rows + 3) / 4));
  const int K = ln_chunks(features);
  bf16* lp = (bf16*)y_lp;
  ESA_TIMED(esa_profile::kLayerNormFwd, st, {
    if (x_dtype == ESA_F32) {
      if (!y || y_dtype == ESA_F32)
        ln_fwd_go(K, grid, st, (const float*)x, weight, bias, rows, features, eps, (float*)y, lp, mean, rstd);
      else
        ln_fwd_go(K, grid, st, (const float*)x, weight, bias, rows, features, eps, (bf16*)y, lp, mean, rstd);
    } else {
      if (!y || y_dtype == ESA_F32)
        ln_fwd_go(K, grid, st, (const bf16*)x, weight, bias, rows, features, eps, (float*)y, lp, mean, rstd);
      else
        ln_fwd_go(K, grid, st, (const bf16*)x, weight, bias, rows, features, eps, (bf16*)y, lp, mean, rstd);
    }
  });
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

extern "C" ESA_API int esa_layer_norm_bwd_workspace_size(int64_t rows, int features, size_t* bytes) {
  if (!bytes) return ESA_ERR_NULL;
  if (rows < 0 || features < 4 || features > kLnMaxFeatures || features % 4) return ESA_ERR_SHAPE;
  *bytes = ((size_t)ln_bwd_blocks(rows) * 2 * features + reduce_scratch_floats(2 * features)) * sizeof(float);
  return ESA_OK;
}

extern "C" ESA_API int esa_layer_norm_bwd(const void* x, int x_dtype, const float* weight, const float* mean,
                                          const float* rstd, const void* dy, int dy_dtype, const void* dy_lp,
                                          const void* dx_add, int64_t rows, int features, void* dx,
                                          float* dweight, float* dbias,
                                          void* workspace, size_t workspace_bytes, void* stream) {
  if (rows < 0 || features < 4 || features > kLnMaxFeatures || features % 4) return ESA_ERR_SHAPE;
  if ((x_dtype != ESA_F32 && x_dtype != ESA_BF16) || (dy && dy_dtype != ESA_F32 && dy_dtype != ESA_BF16))
    return ESA_ERR_DTYPE;
  const bool params = dweight || dbias;
  const size_t need = params ? ((size_t)ln_bwd_blocks(rows) * 2 * features + reduce_scratch_floats(2 * features)) *
                                    sizeof(float)
                              : 0;
  if (params && (!workspace || workspace_bytes < need)) return ESA_ERR_WORKSPACE;
  if (!aligned16(workspace)) return ESA_ERR_ALIGN;
  if (rows == 0) {   // empty input: zero parameter gradients (the reduction over no partials)
    if (params) {
      reduce_columns(nullptr, 0, 2 * features, (float*)workspace, features, dweight, dbias, (hipStream_t)stream);
      ESA_LAUNCH_CHECK();
    }
    return ESA_OK;
  }
  if (!x || !mean || !rstd || !dx || (!dy && !dy_lp)) return ESA_ERR_NULL;
  if (!aligned16(x) || !aligned16(weight) || !aligned16(dy) || !aligned16(dy_lp) || !aligned16(dx) ||
      !aligned16(dx_add))
    return ESA_ERR_ALIGN;
  const int blocks = ln_bwd_blocks(rows);
  float* part = params ? (float*)workspace : nullptr;
  hipStream_t st = (hipStream_t)stream;
  const int K = ln_chunks(features);
  const bf16* lp = (const bf16*)dy_lp;
  ESA_TIMED(esa_profile::kLayerNormBwd, st, {
    const dim3 grid((unsigned)blocks);
    if (x_dtype == ESA_F32) {
      const float* ra = (const float*)dx_add;
      if (!dy || dy_dtype == ESA_F32)
        ln_bwd_go(K, grid, st, (const float*)x, weight, mean, rstd, (const float*)dy, lp, ra, rows, features,
                  (float*)dx, part);
      else
        ln_bwd_go(K, grid, st, (const float*)x, weight, mean, rstd, (const bf16*)dy, lp, ra, rows, features,
                  (float*)dx, part);
    } else {
      const bf16* ra = (const bf16*)dx_add;
      if (!dy || dy_dtype == ESA_F32)
        ln_bwd_go(K, grid, st, (const bf16*)x, weight, mean, rstd, (const float*)dy, lp, ra, rows, features,
                  (bf16*)dx, part);
      else
        ln_bwd_go(K, grid, st, (const bf16*)x, weight, mean, rstd, (const bf16*)dy, lp, ra, rows, features,
                  (bf16*)dx, part);
    }
    if (params)
      reduce_columns(part, blocks, 2 * features, part + (size_t)blocks * 2 * features, features, dweight, dbias, st);
  });
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

extern "C" ESA_API int esa_column_sum_workspace_size(int64_t rows, int cols, size_t* bytes) {
  if (!bytes) return ESA_ERR_NULL;
  if (rows < 0 || cols < 4 || cols % 4) return ESA_ERR_SHAPE;
  *bytes = ((size_t)colsum_row_blocks(rows, cols) * cols + reduce_scratch_floats(cols)) * sizeof(float);
  return ESA_OK;
}

extern "C" ESA_API int esa_column_sum(const void* x, int dtype, int64_t rows, int cols, float* out, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  if (rows < 0 || cols < 4 || cols % 4) return ESA_ERR_SHAPE;
  if (dtype != ESA_F32 && dtype != ESA_BF16) return ESA_ERR_DTYPE;
  if (!out || !workspace || (rows > 0 && !x)) return ESA_ERR_NULL;
  const int rb = colsum_row_blocks(rows, cols);
  if (workspace_bytes < ((size_t)rb * cols + reduce_scratch_floats(cols)) * sizeof(float)) return ESA_ERR_WORKSPACE;
  if (!aligned16(x) || !aligned16(workspace)) return ESA_ERR_ALIGN;
  hipStream_t st = (hipStream_t)stream;
  float* part = (float*)workspace;
  ESA_TIMED(esa_profile::kColumnSum, st, {
    if (rows > 0) {
      const int chunks = cols / 4;
      const int tpb = std::min(256, (chunks + 63) / 64 * 64);
      const dim3 grid((unsigned)((chunks + tpb - 1) / tpb), (unsigned)rb);
      const int64_t rpb = (rows + rb - 1) / rb;
      if (dtype == ESA_F32)
        hipLaunchKernelGGL(col_sum_partial_kernel<float>, grid, dim3(tpb), 0, st, (const float*)x, rows, cols, rpb,
                           part);
      else
        hipLaunchKernelGGL(col_sum_partial_kernel<bf16>, grid, dim3(tpb), 0, st, (const bf16*)x, rows, cols, rpb,
                           part);
    }
    reduce_columns(part, rows > 0 ? rb : 0, cols, part + (size_t)rb * cols, cols, out, nullptr, st);
  });
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

extern "C" ESA_API int esa_mish_bwd_colsum(const void* z, const void* grad, int64_t rows, int cols, int dtype,
                                           void* dz, float* dbias, void* workspace, size_t workspace_bytes,
                                           void* stream) {
  if (rows < 0 || cols < 4 || cols % 4) return ESA_ERR_SHAPE;
  if (dtype != ESA_F32 && dtype != ESA_BF16) return ESA_ERR_DTYPE;
  if (!dbias || !workspace || (rows > 0 && (!z || !grad || !dz))) return ESA_ERR_NULL;
  const int rb = colsum_row_blocks(rows, cols);
  if (workspace_bytes < ((size_t)rb * cols + reduce_scratch_floats(cols)) * sizeof(float)) return ESA_ERR_WORKSPACE;
  if (!aligned16(z) || !aligned16(grad) || !aligned16(dz) || !aligned16(workspace)) return ESA_ERR_ALIGN;
  hipStream_t st = (hipStream_t)stream;
  float* part = (float*)workspace;
  ESA_TIMED(esa_profile::kMishBwd, st, {
    if (rows > 0) {
      const int cpt = dtype == ESA_BF16 && cols % 8 == 0 ? 8 : 4;   // one 16-byte access per row and thread
      const int chunks = cols / cpt;
      const int tpb = std::min(256, (chunks + 63) / 64 * 64);
      const dim3 grid((unsigned)((chunks + tpb - 1) / tpb), (unsigned)rb);
      const int64_t rpb = (rows + rb - 1) / rb;
      if (dtype == ESA_F32)
        hipLaunchKernelGGL((mish_bwd_colsum_kernel<float, 4>), grid, dim3(tpb), 0, st, (const float*)z,
                           (const float*)grad, rows, cols, rpb, (float*)dz, part);
      else if (cpt == 8)
        hipLaunchKernelGGL((mish_bwd_colsum_kernel<bf16, 8>), grid, dim3(tpb), 0, st, (const bf16*)z,
                           (const bf16*)grad, rows, cols, rpb, (bf16*)dz, part);
      else
        hipLaunchKernelGGL((mish_bwd_colsum_kernel<bf16, 4>), grid, dim3(tpb), 0, st, (const bf16*)z,
                           (const bf16*)grad, rows, cols, rpb, (bf16*)dz, part);
    }
    reduce_columns(part, rows > 0 ? rb : 0, cols, part + (size_t)rb * cols, cols, dbias, nullptr, st);
  });
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

extern "C" ESA_API int esa_mab_residual_fwd(const void* z, const void* o, const float* x, int64_t n, int dtype,
                                            float* y, void* stream) {
  if (n < 0) return ESA_ERR_SHAPE;
  if (dtype != ESA_F32 && dtype != ESA_BF16) return ESA_ERR_DTYPE;
  if (n == 0) return ESA_OK;
  if (!z || !o || !x || !y) return ESA_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == ESA_F32) return mab_residual_fwd_typed((const float*)z, (const float*)o, x, y, n, st);
  return mab_residual_fwd_typed((const bf16*)z, (const bf16*)o, x, y, n, st);
}

extern "C" ESA_API int esa_mab_residual_bwd(const void* z, const float* g, int64_t n, int dtype, void* dz, void* g_o,
                                            void* stream) {
  if (n < 0) return ESA_ERR_SHAPE;
  if (dtype != ESA_F32 && dtype != ESA_BF16) return ESA_ERR_DTYPE;
  if (n == 0) return ESA_OK;
  if (!z || !g || !dz || !g_o) return ESA_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == ESA_F32) return mab_residual_bwd_typed((const float*)z, g, (float*)dz, (float*)g_o, n, st);
  return mab_residual_bwd_typed((const bf16*)z, g, (bf16*)dz, (bf16*)g_o, n, st);
}

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
