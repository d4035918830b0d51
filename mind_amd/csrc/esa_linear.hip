// fp32 Linear layers of the packed ESA blocks on gfx950: y_i = x W_i^T + b_i
// for up to three (W_i, b_i) over one input x [rows, K] in one launch (the
// MAB's fc_q / fc_k / fc_v share their input, esa/mha.py:54-56, and the
// PMA's fc_k / fc_v theirs).  The reference runs them as three nn.Linear
// calls in fp32 (configuration 0's modules).  On packed tokens the shapes
// are tall and narrow (rows = tokens, K and N of 128-512) and a GEMM of
// 21,752 x 128 x 128 is latency-bound: hipBLASLt's kernel and this one
// both take about 20 us per weight on the GPU.  One launch over the three
// weights fills the chip three times as densely: 41.8 us against 57.3 us
// for three library calls (configuration 0's fc_q / fc_k / fc_v, timed in
// a HIP graph).  Single weights stay with the library GEMM, which is as
// fast at N = 128 and twice as fast at N = 256 (a tile over all 256
// columns reads x once).
//
// One wave computes a 64 x 64 tile of one output (4 x 4 blocks of 16 x 16)
// with v_mfma_f32_16x16x4_f32 over the whole K: per 16-k chunk a lane loads
// one float4 of each of its four x rows and four W rows straight from L2
// (both tensors row-major with k innermost, so a 16-k chunk of 16 rows is 64
// contiguous bytes per row), and the four MFMAs of a block pair take k
// offsets u = 0..3 of every lane's float4: MFMA u sums the products at k =
// kb + 4g + u over the lane groups g = lane / 16, which covers the chunk.
// Eight 16-byte loads per lane feed 64 MFMAs; with 16-row tiles the same
// chunk took five loads per 16 MFMAs and the weight rows, re-read for every
// 16 rows, bounded the kernel at a fifth of the MFMA rate.  The next chunk's
// loads are issued before the current chunk's MFMAs.  The epilogue adds the
// bias and stores fp32 rows (64 contiguous bytes per row segment).  Work
// items are (64-row block, 64-column tile) pairs, column tile fastest, four
// per hardware block; the hardware block order is remapped so that each XCD
// takes a contiguous range of items and the column tiles of one row block
// (which read the same x rows) share its L2.
//
// fp32 MFMA multiplies exactly and accumulates in fp32; the summation order
// differs from a library GEMM's, so results agree with torch's F.linear to
// fp32 rounding (a few ulp relative), not bit for bit.
#include "esa_common.h"
#include "esa_profile.h"
#include "../../include/esa_hip.h"

namespace {

constexpr int kMaxOut = 3;
constexpr int kRowTiles = 4, kColTiles = 4;   // 16 x 16 blocks per wave along rows / columns
constexpr int kRowsPerWave = 16 * kRowTiles, kWaves = 4, kColsPerWave = 16 * kColTiles, kChunk = 16;

struct LinearOut {
  const float* w; const float* b; float* y;
  int n;       // out_features (multiple of 64)
  int tile0;   // first column tile of this output among all outputs' tiles
};

struct LinearArgs {
  const float* x;
  int rows, k, n_out, col_tiles, row_blocks;
  LinearOut out[kMaxOut];
};

// D(16x16, fp32) += A(16x4) B(4x16): lane l supplies A[l%16][l/16] and
// B[l/16][l%16]; it receives D[4(l/16) + r][l%16] in accumulator register r.
DEVI f32x4 mfma16x4(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

DEVI float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

__global__ __launch_bounds__(256) void linear_f32_kernel(const LinearArgs a) {
  // XCD-contiguous order: hardware block h runs on XCD h mod 8; block index
  // v gives each XCD a contiguous range; wave item = 4 v + wave.
  const int G = (int)gridDim.x, h = (int)blockIdx.x, xcd = h & 7, q = G >> 3, rem = G & 7;
  const int v = xcd * q + min(xcd, rem) + (h >> 3);
  const int item = v * kWaves + (int)(threadIdx.x >> 6);
  const int rb = item / a.col_tiles, ct = item - rb * a.col_tiles;
  const int lane = threadIdx.x & 63;
  const int row0 = rb * kRowsPerWave;
  if (row0 >= a.rows) return;   // wave-uniform; the kernel has no barriers
  int o = 0;
#pragma unroll
  for (int i = 1; i < kMaxOut; ++i)
    if (i < a.n_out && ct >= a.out[i].tile0) o = i;
  const LinearOut out = a.out[o];
  const int col0 = (ct - out.tile0) * kColsPerWave;
  const int r = lane & 15, g = lane >> 4, K = a.k;
  const float* xp[kRowTiles];
  const float* wp[kColTiles];
#pragma unroll
  for (int t = 0; t < kRowTiles; ++t)   // rows past the end re-read the last
    xp[t] = a.x + (size_t)min(row0 + 16 * t + r, a.rows - 1) * K + 4 * g;
#pragma unroll
  for (int t = 0; t < kColTiles; ++t) wp[t] = out.w + (size_t)(col0 + 16 * t + r) * K + 4 * g;
  f32x4 acc[kRowTiles][kColTiles];
#pragma unroll
  for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
    for (int j = 0; j < kColTiles; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Two register buffers: chunk kb + 16 loads while chunk kb multiplies.
  float4 xa[2][kRowTiles], wb[2][kColTiles];
  auto load = [&](int buf, int kb) {
#pragma unroll
    for (int t = 0; t < kRowTiles; ++t) xa[buf][t] = ld4(xp[t] + kb);
#pragma unroll
    for (int t = 0; t < kColTiles; ++t) wb[buf][t] = ld4(wp[t] + kb);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto multiply = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
        for (int j = 0; j < kColTiles; ++j)
          acc[i][j] = mfma16x4(xa[buf][i][u], wb[buf][j][u], acc[i][j]);
  };
  // Loads past the last chunk re-read it (unconditional loads keep the waits
  // exact: each multiply waits only for its own buffer).
  load(0, 0);
  for (int kb = 0; kb < K; kb += 2 * kChunk) {
    load(1, min(kb + kChunk, K - kChunk));
    multiply(0);
    if (kb + kChunk >= K) break;   // odd chunk count: the last chunk was in buffer 0
    load(0, min(kb + 2 * kChunk, K - kChunk));
    multiply(1);
  }
#pragma unroll
  for (int j = 0; j < kColTiles; ++j) {
    const int col = col0 + 16 * j + r;
    const float bias = out.b ? out.b[col] : 0.f;
#pragma unroll
    for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = row0 + 16 * i + 4 * g + e;
        if (row < a.rows) out.y[(size_t)row * out.n + col] = acc[i][j][e] + bias;
      }
  }
}

bool misaligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) != 0; }

}  // namespace

extern "C" {

int esa_linear_f32(const float* x, int rows, int in_features, int n_out, const float* const* weight,
                   const float* const* bias, float* const* y, const int* out_features, void* stream) {
  if (n_out < 1 || n_out > kMaxOut) return ESA_ERR_SHAPE;
  if (!weight || !bias || !y || !out_features) return ESA_ERR_NULL;
  if (rows < 0 || in_features < kChunk || in_features % kChunk) return ESA_ERR_SHAPE;
  LinearArgs a{};
  a.x = x; a.rows = rows; a.k = in_features; a.n_out = n_out;
  int tiles = 0;
  for (int i = 0; i < n_out; ++i) {
    const int n = out_features[i];
    if (n < kColsPerWave || n % kColsPerWave) return ESA_ERR_SHAPE;
    a.out[i] = LinearOut{weight[i], bias[i], y[i], n, tiles};
    tiles += n / kColsPerWave;
  }
  if (rows == 0) return ESA_OK;   // nothing to read or write: empty tensors may have null pointers
  if (!x) return ESA_ERR_NULL;
  if (misaligned16(x)) return ESA_ERR_ALIGN;
  for (int i = 0; i < n_out; ++i) {
    if (!weight[i] || !y[i]) return ESA_ERR_NULL;
    if (misaligned16(weight[i]) || misaligned16(y[i])) return ESA_ERR_ALIGN;
  }
  a.col_tiles = tiles;
  a.row_blocks = (rows + kRowsPerWave - 1) / kRowsPerWave;
  const long long items = (long long)a.row_blocks * tiles, blocks = (items + kWaves - 1) / kWaves;
  if (blocks > 0x7fffffffLL) return ESA_ERR_SHAPE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  ESA_TIMED(esa_profile::kLinearF32, st,
            hipLaunchKernelGGL(linear_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

}  // extern "C"
