// Tile constants and device helpers shared by the bf16 attention kernels
// (the edge-mask walks in esa_attn.hip, the segment-tiled dense kernels in
// esa_attn_dense.hip): MFMA operand layouts, LDS layouts, bf16 splits.
#pragma once
#include <climits>

#include "esa_common.h"

namespace {

constexpr int kTile = 32;
constexpr int kHd = 16;
constexpr int kWaves = 4;
constexpr int kGroupTok = kWaves * kTile;   // 128 tokens per block
constexpr int kRowStride = 24;              // bf16 per row of a [32 tokens][16] LDS tile (48 B)
constexpr int kTrStride = 40;               // bf16 per row of a [rows][32 tokens] LDS tile (80 B)
constexpr float kStaticBound = 60.f;
constexpr float kDeadRow = -1.0e30f;        // -LSE2/c for rows without keys: every exp2 underflows to 0

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef int i32x4 __attribute__((ext_vector_type(4)));

DEVI i32x4 bload(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0); }
DEVI bf16x8 as_bf16x8(i32x4 v) { return __builtin_bit_cast(bf16x8, v); }

DEVI int kperm(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }

DEVI bool node_adjacent(int2 a, int2 b) {
  return (a.x == b.x) | (a.x == b.y) | (a.y == b.x) | (a.y == b.y);
}

// Conservative tile-pair test for the edge mask: node-id ranges must overlap
// and the 64-bit node signatures (bit n & 63) must intersect.
DEVI bool tiles_may_touch(int4 a, int4 b) {
  if (a.y < b.x || b.y < a.x) return false;
  return ((a.z & b.z) | (a.w & b.w)) != 0;
}
DEVI int4 no_touch() { return make_int4(INT_MAX, INT_MIN, 0, 0); }

DEVI float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

DEVI void store_rows8(bf16* __restrict__ dst, const f32x16& acc, float mul, int half) {
  bf16x4 o0, o1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o0[i] = (bf16)(acc[i] * mul);
    o1[i] = (bf16)(acc[4 + i] * mul);
  }
  *reinterpret_cast<bf16x4*>(dst + 4 * half) = o0;
  *reinterpret_cast<bf16x4*>(dst + 8 + 4 * half) = o1;
}

DEVI bf16x8 cvt8(const float* p) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (bf16)p[e];
  return r;
}

DEVI bf16x8 lds8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }

// c * x as an unevaluated pair of bf16 vectors (hi + lo carries ~16
// significant bits): two MFMAs with hi and lo give c * (a . x) in fp32
// without a VALU multiply per score.
DEVI void split_scaled(const bf16x8& x, float c, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float v = (float)x[e] * c;
    hi[e] = (bf16)v;
    lo[e] = (bf16)(v - (float)hi[e]);
  }
}

// ---- 16x16 block layouts (dense backward kernels)
// A 32x32 (partner x owned) tile is four 16x16 blocks.  The score MFMA
// (mfma16k32) gives lane l partner rows 4G..4G+3 (G = l / 16) of a block
// for owned token l % 16, so the tile's two partner blocks leave a lane 8
// partner rows of one owned token, {4G..4G+3, 16+4G..16+4G+3}: exactly the
// K slots 8G..8G+7 a lane supplies to the mfma16k32 that sums over the
// tile's 32 partners.  slot_col(t) is the K slot of tile-local partner t
// in that order; tr_operand (below) reads the matching A operand.
DEVI int slot_col(int t) { return 8 * ((t & 15) >> 2) + 4 * (t >> 4) + (t & 3); }

// B operand of a scaled score mfma16k32: K slots 0..15 carry the bf16 hi
// halves of c * x, slots 16..31 the lo halves (hi + lo carries ~16
// significant bits), so one MFMA gives c * (a . x) in fp32.  Lane group G
// supplies slots 8G..8G+7: x holds dims 8 (G & 1)..+7 and lo = (G >= 2).
DEVI bf16x8 scaled_half(const bf16x8& x, float c, bool lo) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float v = (float)x[e] * c;
    const bf16 hi = (bf16)v;
    r[e] = lo ? (bf16)(v - (float)hi) : hi;
  }
  return r;
}

// B operand over a tile's 32 partners from the two partner blocks' results.
DEVI bf16x8 cvt4x2(const f32x4& a, const f32x4& b) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r[e] = (bf16)a[e];
    r[4 + e] = (bf16)b[e];
  }
  return r;
}

DEVI f32x4 splat4(float x) { return f32x4{x, x, x, x}; }
DEVI bf16x4 lds4(const bf16* p) { return *reinterpret_cast<const bf16x4*>(p); }
DEVI f32x4 ldsf4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

// dims 4g..4g+3 of one token row: mul * acc (an mfma16k* result column).
DEVI void store_dims4(bf16* __restrict__ row, const f32x4& acc, float mul, int g) {
  bf16x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = (bf16)(acc[i] * mul);
  *reinterpret_cast<bf16x4*>(row + 4 * g) = o;
}

// ---- staged rows split by dims half
// An LDS tile of token rows as two [n][8] bf16 arrays (dims 0..7, 8..15),
// HS bf16 apart: the 16 lanes of a lane group reading 16 consecutive
// tokens' halves touch 256 contiguous bytes (no bank conflicts on gfx950).
template <int HS>
DEVI void put_half(bf16* rows, int tok, int h, i32x4 v) {
  *reinterpret_cast<i32x4*>(&rows[h * HS + tok * 8]) = v;
}
template <int HS>
DEVI bf16x8 half_row8(const bf16* rows, int tok, int h) { return lds8(&rows[h * HS + tok * 8]); }
template <int HS>
DEVI bf16x4 half_row4(const bf16* rows, int tok, int q) {   // dims 4q .. 4q + 3
  return lds4(&rows[(q >> 1) * HS + tok * 8 + 4 * (q & 1)]);
}

// ds_read_b64_tr_b16 (gfx950): lane i of a 16-lane group receives, as its
// element k, element i % 4 of the 8-byte chunk addressed by lane 4k + i / 4
// of the group.
DEVI bf16x4 lds_tr4(const bf16* p) {
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p);
}

// The mfma16k32 A operand over the 32 tokens of a split-row tile starting at
// token t0 (lane c16 + 16 grp: dim c16 of the tokens in K slots 8 grp ..
// 8 grp + 7, slot order of slot_col) by two transpose reads: lane j of the
// group addresses token 4 grp + j / 4 (16 more for the second read), dims
// 4 (j % 4) .. +3, so lane i receives dim i of four tokens.
template <int HS>
DEVI bf16x8 tr_operand(const bf16* rows, int t0, int c16, int grp) {
  const int q = c16 & 3;
  const bf16* p = rows + (q >> 1) * HS + (t0 + 4 * grp + (c16 >> 2)) * 8 + 4 * (q & 1);
  const bf16x4 lo = lds_tr4(p), hi = lds_tr4(p + 16 * 8);
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// A operands of the two mfma32 products that sum over the 32 tokens of a
// split-row tile at token t0 (K slots = tokens 0..15, then 16..31; A rows =
// the 16 dims), by transpose reads.  Lane groups 0 and 2 (rows 0..15, K
// slots 0..7 and 8..15) read dims of four tokens per read.  Groups 1 and 3
// (rows 16..31) read the 4-element array `ones` when it is given (the ones
// rows of [V^T ; 1], whose product is the softmax row sum), else the same
// dims again (rows 16..31 duplicate rows 0..15).
template <int HS>
DEVI void tr_rows32(const bf16* rows, int t0, const bf16* ones, int c16, int grp, bf16x8& op0, bf16x8& op1) {
  const int q = c16 & 3;
  const bool one = ones && (grp & 1);
  const int step = one ? 0 : 8;   // bf16 per token in the read address
  const bf16* p = one ? ones : rows + (q >> 1) * HS + (t0 + 8 * (grp >> 1) + (c16 >> 2)) * 8 + 4 * (q & 1);
  const bf16x4 v0 = lds_tr4(p), v1 = lds_tr4(p + 4 * step);
  const bf16x4 v2 = lds_tr4(p + 16 * step), v3 = lds_tr4(p + 20 * step);
  op0 = bf16x8{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
  op1 = bf16x8{v2[0], v2[1], v2[2], v2[3], v3[0], v3[1], v3[2], v3[3]};
}

DEVI f32x16 splat16(float x) {
  f32x16 r;
#pragma unroll
  for (int i = 0; i < 16; ++i) r[i] = x;
  return r;
}

// Node pairs of the 16 partner tokens of a half-wave's accumulator rows
// (tile-local 16(r>>3) + 8h + (r&7)), from an LDS tile of 32 node pairs.
DEVI void lds_nodes16(const int2* sn, int half, int2 out[16]) {
  const int4* p0 = reinterpret_cast<const int4*>(sn + 8 * half);
  const int4* p1 = reinterpret_cast<const int4*>(sn + 16 + 8 * half);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int4 a = p0[j], b = p1[j];
    out[2 * j] = make_int2(a.x, a.y);
    out[2 * j + 1] = make_int2(a.z, a.w);
    out[8 + 2 * j] = make_int2(b.x, b.y);
    out[8 + 2 * j + 1] = make_int2(b.z, b.w);
  }
}

DEVI int row_local(int r, int half) { return 16 * (r >> 3) + 8 * half + (r & 7); }

// max |k_t| over one 32-token key tile, per head: knorm[h * n_tiles + tile].
// Consecutive threads read consecutive heads of a token (contiguous rows).
DEVI void knorm_block(const bf16* __restrict__ k, int total, int heads, int n_tiles, float* __restrict__ knorm,
                      int tile, int tid) {
  __shared__ int smax[256];
  for (int h0 = 0; h0 < heads; h0 += 256) {
    const int hn = min(256, heads - h0);
    if (tid < hn) smax[tid] = 0;
    __syncthreads();
    for (int i = tid; i < kTile * hn; i += 256) {
      const int t = tile * kTile + i / hn, h = h0 + i % hn;
      if (t < total) {
        const bf16x8* p = reinterpret_cast<const bf16x8*>(k + ((size_t)t * heads + h) * kHd);
        const bf16x8 u = p[0], v = p[1];
        float x = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) x = fmaf((float)u[e], (float)u[e], fmaf((float)v[e], (float)v[e], x));
        atomicMax(&smax[h - h0], __float_as_int(x));   // x >= 0: int order is float order
      }
    }
    __syncthreads();
    if (tid < hn) knorm[(size_t)(h0 + tid) * n_tiles + tile] = sqrtf(__int_as_float(smax[tid]));
    __syncthreads();
  }
}

DEVI uint32_t split_bf16_pair(float x) {
  const bf16 hi = (bf16)x;
  const bf16 lo = (bf16)(x - (float)hi);
  return (uint32_t)__builtin_bit_cast(uint16_t, hi) | ((uint32_t)__builtin_bit_cast(uint16_t, lo) << 16);
}

// ---- LDS-direct staging (list kernels, dense dK/dV)
// buffer_load_dwordx4 / _dword with the LDS flag: lane l's 16 (4) bytes land
// at M0 + 16 l (4 l), so a split-row tile (lane = token col of dims half l >> 5)
// stages with one instruction per head and tensor and no staging registers.
// Loads past the buffer range write zeros.  Issued as assembly: the
// compiler's wait-count pass does not see them (its own waits only get more
// conservative), and the stage loop waits for them explicitly.  M0 is set
// right before each load (one SALU wait state); nothing else in these
// kernels uses M0.
DEVI uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p);
}
DEVI void dma16(rsrc_t r, uint32_t off, const void* lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds" ::"v"(off), "s"(lds_addr(lds)),
               "s"(r)
               : "memory");
}
DEVI void dma4(rsrc_t r, uint32_t off, const void* lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dword %0, %2, 0 offen lds" ::"v"(off), "s"(lds_addr(lds)),
               "s"(r)
               : "memory");
}
// s_waitcnt vmcnt(n) (gfx9 encoding: vmcnt bits 3:0 and 15:14; expcnt and
// lgkmcnt at their maxima, i.e. not waited for).
template <int N>
DEVI void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// ---- per-segment work plans (dense bf16 and fp32 attention kernels)
// Groups of one direction: every segment's outer tokens cut into groups of
// `gtok` tokens (one block each), segments ordered by partner tiles (longest first, counting sort in
// one block; segments with equal counts in any order, which changes no
// result).  groups[i] = (outer begin, outer segment end, inner begin, inner end).
constexpr int kPlanBuckets = 1024;

DEVI void seg_plan_block(const int* __restrict__ cu_outer, const int* __restrict__ cu_inner, int nseg, int gtok,
                         int4* __restrict__ groups, int* __restrict__ count, int tid) {
  constexpr int PER = kPlanBuckets / 256;
  __shared__ int hist[kPlanBuckets];
  __shared__ int part[256];
  for (int i = tid; i < kPlanBuckets; i += 256) hist[i] = 0;
  __syncthreads();
  auto bucket = [&](int s) {
    const int tiles = (cu_inner[s + 1] - cu_inner[s] + kTile - 1) / kTile;
    return kPlanBuckets - 1 - min(max(tiles, 0), kPlanBuckets - 1);
  };
  for (int s = tid; s < nseg; s += 256) {
    const int n = cu_outer[s + 1] - cu_outer[s];
    if (n > 0) atomicAdd(&hist[bucket(s)], (n + gtok - 1) / gtok);
  }
  __syncthreads();
  int loc[PER], sum = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    loc[i] = sum;
    sum += hist[tid * PER + i];
  }
  part[tid] = sum;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int add = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += add;
    __syncthreads();
  }
  const int base = part[tid] - sum;
#pragma unroll
  for (int i = 0; i < PER; ++i) hist[tid * PER + i] = base + loc[i];
  if (tid == 255) *count = part[255];
  __syncthreads();
  for (int s = tid; s < nseg; s += 256) {
    const int ob = cu_outer[s], oe = cu_outer[s + 1];
    if (oe <= ob) continue;
    const int ng = (oe - ob + gtok - 1) / gtok;
    const int pos = atomicAdd(&hist[bucket(s)], ng);
    const int ib = cu_inner[s], ie = cu_inner[s + 1];
    for (int j = 0; j < ng; ++j) groups[pos + j] = make_int4(ob + j * gtok, oe, ib, max(ie, ib));
  }
}

}  // namespace
