// Varlen (packed-segment) attention for edge-set attention on gfx950.
//
// Forward:  O = softmax(scale * Q K^T + mask) V per segment, fp32 softmax,
//           bf16 MFMA (v_mfma_f32_32x32x16_bf16) for Q K^T and P V.
// Backward: two deterministic passes (no atomics):
//           K-outer pass -> dK, dV;  Q-outer pass -> dQ.
//
// Semantics follow flash_attn_varlen_func as called at
// esa/mha_flash_varlen.py:177-184 (causal=False, dropout 0), and, with the
// edge-adjacency mask, the additive 0/-99999 bias that
// get_adj_mask_from_edge_index_edge builds (esa/masked_layers.py:121-142,
// 217-268) and memory_efficient_attention applies (esa/mha.py:73-77).
//
// Tiling.  Tokens are cut into 32-token tiles aligned to the global token
// index, so every vector load is aligned; a tile may straddle segments, which
// the per-element validity test (key in the query's segment) resolves.  One
// wave computes one (32-token tile, head) pair; a 256-thread block holds four
// heads of the same tile.  Tiles are dispatched longest-first (a per-call
// plan kernel sorts them by the number of partner tiles).
//
// Register layout (head_dim = 16 = the MFMA K of 32x32x16):
//   S^T = K_tile * Q_tile^T : lane l owns query column l%32; its 16 fp32
//   accumulators hold keys k0 + 16(r>>3) + 8(l>>5) + (r&7).  Rows of the K
//   operand are permuted (bits 2 and 3 of the row swapped) to make that
//   mapping, so each half-wave's 8 P values are 8 consecutive keys — exactly
//   the B operand of the P V product, with no data movement.
//   O^T = [V^T ; 1] * P^T : rows 0..15 are the output dims, rows 16..31 are
//   ones, so the MFMA also produces the softmax row sum.  Softmax statistics
//   stay per lane (one query per lane; the two half-waves exchange one max).
//   V^T (and K^T, Q^T, dO^T in backward) is pre-transposed into a
//   tile-transposed layout [T/8][H][16][8] so each lane's A operand is one
//   aligned 16-byte load.
#include "esa_common.h"
#include "esa_profile.h"
#include "../../include/esa_hip.h"

namespace {

constexpr int kTile = 32;
constexpr int kHd = 16;

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

// Node pairs of the 16 tokens a half-wave's accumulator rows refer to:
// tokens base + 8h + 0..7 and base + 16 + 8h + 0..7.
DEVI void load_nodes16(const int2* __restrict__ nodes, int base, int half, int2 out[16]) {
  const int4* p0 = reinterpret_cast<const int4*>(nodes + base + 8 * half);
  const int4* p1 = reinterpret_cast<const int4*>(nodes + base + 16 + 8 * half);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    int4 a = p0[j], b = p1[j];
    out[2 * j] = make_int2(a.x, a.y);
    out[2 * j + 1] = make_int2(a.z, a.w);
    out[8 + 2 * j] = make_int2(b.x, b.y);
    out[8 + 2 * j + 1] = make_int2(b.z, b.w);
  }
}

DEVI int row_token(int base, int r, int half) { return base + 16 * (r >> 3) + 8 * half + (r & 7); }

DEVI bf16x8 splat8(float x) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (bf16)x;
  return r;
}

// A-operand fragment from a tile-transposed [T/8][H][16][8] array: rows are
// the 16 feature dims (lanes with l%32 >= 16 get `fill`), slots are the 8
// tokens starting at chunk `chunk`.
DEVI bf16x8 tt_frag(const bf16* __restrict__ tt, int chunk, int heads, int head, int col, bf16x8 fill) {
  const bf16x8 v = *reinterpret_cast<const bf16x8*>(tt + ((size_t)(chunk * heads + head) * kHd + (col & 15)) * 8);
  return col < 16 ? v : fill;
}

DEVI bf16x8 row_frag(const bf16* __restrict__ x, int token, int heads, int head, int half) {
  return *reinterpret_cast<const bf16x8*>(x + ((size_t)token * heads + head) * kHd + 8 * half);
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

struct QOuterArgs {
  const bf16* q; const bf16* k; const bf16* v;
  const bf16* at;          // forward: V^T (tile-transposed); dQ pass: K^T
  const bf16* dout;        // dQ pass
  const float* lse2;       // dQ pass: log2-domain LSE [H][tq_pad], +inf = dead row
  const float* dvec;       // dQ pass: rowsum(dO * O) [H][tq_pad]
  const int* cu_q; const int* cu_k; int nseg;
  int total_q, total_k, heads, tq_pad;
  float c;                 // softmax_scale * log2(e)
  float scale;
  const int2* nodes; const int4* meta;
  const int* plan; int n_tiles;
  bf16* out; float* lse;   // forward outputs
  bf16* dq;                // dQ pass output
};

// One wave = one (query tile, head).  DQ=false: forward.  DQ=true: dQ pass.
template <bool MASKED, bool DQ>
__global__ __launch_bounds__(256) void attn_qouter_kernel(const QOuterArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int groups = (a.heads + 3) >> 2;
  const int item = blockIdx.x / groups;
  const int head = (blockIdx.x - item * groups) * 4 + wave;
  if (head >= a.heads) return;
  const int H = a.heads;
  const int qt = a.plan[item];
  const int q0 = qt * kTile;
  const int col = lane & 31, half = lane >> 5;
  const int qi = q0 + col;
  const bool qvalid = qi < a.total_q;
  const int qc = qvalid ? qi : a.total_q - 1;
  const int q_last = min(q0 + kTile - 1, a.total_q - 1);
  const int seg_first = seg_of(a.cu_q, a.nseg, q0);
  const int seg_last = seg_of(a.cu_q, a.nseg, q_last);
  const int seg = seg_of(a.cu_q, a.nseg, qc);
  int klo = a.cu_k[seg], khi = a.cu_k[seg + 1];
  if (!qvalid) { klo = 0; khi = 0; }
  const int kbeg = a.cu_k[seg_first], kend = a.cu_k[seg_last + 1];
  const int klo_max = a.cu_k[seg_last], khi_min = a.cu_k[seg_first + 1];

  const bf16x8 qf = row_frag(a.q, qc, H, head, half);
  int2 qn = make_int2(0, 0);
  int4 qmeta = make_int4(0, 0, 0, 0);
  if (MASKED) { qn = a.nodes[qc]; qmeta = a.meta[qt]; }
  bf16x8 dof = splat8(0.f);
  float lse2q = 0.f, dq_d = 0.f;
  if (DQ) {
    dof = row_frag(a.dout, qc, H, head, half);
    lse2q = a.lse2[(size_t)head * a.tq_pad + qc];
    dq_d = a.dvec[(size_t)head * a.tq_pad + qc];
  }
  const bf16x8 fill = splat8(DQ ? 0.f : 1.f);
  const f32x16 zero = {};
  f32x16 acc = {};
  float m_run = -INFINITY;

  const int kt_beg = kbeg >> 5, kt_end = (kend + kTile - 1) >> 5;
  for (int kt = kt_beg; kt < kt_end; ++kt) {
    const int k0 = kt * kTile;
    if (MASKED) {
      if (!tiles_may_touch(qmeta, a.meta[kt])) continue;
    }
    const int kr = min(k0 + kperm(col), a.total_k - 1);
    const bf16x8 kf = row_frag(a.k, kr, H, head, half);
    f32x16 s = mfma32(kf, qf, zero);
    const bool full = !MASKED && k0 >= klo_max && k0 + kTile <= khi_min;
    if (!full) {
      int2 kn[16];
      if (MASKED) load_nodes16(a.nodes, k0, half, kn);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = row_token(k0, r, half);
        bool ok = key >= klo && key < khi;
        if (MASKED) ok = ok && key != qi && node_adjacent(kn[r], qn);
        s[r] = ok ? s[r] : -INFINITY;
      }
    }
    if (!DQ) {
      float mt = s[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
      mt = fmaxf(mt, __shfl_xor(mt, 32));
      const float m_new = fmaxf(m_run, mt * a.c);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = fast_exp2(m_run - m_use);
      m_run = m_new;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] *= alpha;
      bf16x8 p0, p1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p0[e] = (bf16)fast_exp2(fmaf(s[e], a.c, -m_use));
        p1[e] = (bf16)fast_exp2(fmaf(s[8 + e], a.c, -m_use));
      }
      const bf16x8 v0 = tt_frag(a.at, (k0 >> 3) + half, H, head, col, fill);
      const bf16x8 v1 = tt_frag(a.at, (k0 >> 3) + 2 + half, H, head, col, fill);
      acc = mfma32(v0, p0, acc);
      acc = mfma32(v1, p1, acc);
    } else {
      const bf16x8 vf = row_frag(a.v, kr, H, head, half);
      const f32x16 dp = mfma32(vf, dof, zero);
      bf16x8 d0, d1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float p0 = fast_exp2(fmaf(s[e], a.c, -lse2q));
        const float p1 = fast_exp2(fmaf(s[8 + e], a.c, -lse2q));
        d0[e] = (bf16)(p0 * (dp[e] - dq_d));
        d1[e] = (bf16)(p1 * (dp[8 + e] - dq_d));
      }
      const bf16x8 k0f = tt_frag(a.at, (k0 >> 3) + half, H, head, col, fill);
      const bf16x8 k1f = tt_frag(a.at, (k0 >> 3) + 2 + half, H, head, col, fill);
      acc = mfma32(k0f, d0, acc);
      acc = mfma32(k1f, d1, acc);
    }
  }

  if (!qvalid) return;
  if (!DQ) {
    const float l = acc[8];  // a ones row of [V^T; 1] P^T: the softmax row sum
    const float inv = l > 0.f ? 1.f / l : 0.f;
    store_rows8(a.out + ((size_t)qi * H + head) * kHd, acc, inv, half);
    if (half == 0)
      a.lse[(size_t)head * a.total_q + qi] = l > 0.f ? (m_run + fast_log2(l)) * kLn2 : -INFINITY;
  } else {
    store_rows8(a.dq + ((size_t)qi * H + head) * kHd, acc, a.scale, half);
  }
}

struct KOuterArgs {
  const bf16* q; const bf16* k; const bf16* v; const bf16* dout;
  const bf16* qt; const bf16* dot;   // tile-transposed Q and dO
  const float* lse2; const float* dvec;
  const int* cu_q; const int* cu_k; int nseg;
  int total_q, total_k, heads, tq_pad;
  float c, scale;
  const int2* nodes; const int4* meta;
  const int* plan; int n_tiles;
  bf16* dk; bf16* dv;
};

// One wave = one (key tile, head): dV = P^T dO and dK = scale * dS^T Q,
// accumulated over every query tile of the key tile's segments.
template <bool MASKED>
__global__ __launch_bounds__(256) void attn_kouter_kernel(const KOuterArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int groups = (a.heads + 3) >> 2;
  const int item = blockIdx.x / groups;
  const int head = (blockIdx.x - item * groups) * 4 + wave;
  if (head >= a.heads) return;
  const int H = a.heads;
  const int kt = a.plan[item];
  const int k0 = kt * kTile;
  const int col = lane & 31, half = lane >> 5;
  const int ki = k0 + col;
  const bool kvalid = ki < a.total_k;
  const int kc = kvalid ? ki : a.total_k - 1;
  const int k_last = min(k0 + kTile - 1, a.total_k - 1);
  const int seg_first = seg_of(a.cu_k, a.nseg, k0);
  const int seg_last = seg_of(a.cu_k, a.nseg, k_last);
  const int seg = seg_of(a.cu_k, a.nseg, kc);
  int qlo = a.cu_q[seg], qhi = a.cu_q[seg + 1];
  if (!kvalid) { qlo = 0; qhi = 0; }
  const int qbeg = a.cu_q[seg_first], qend = a.cu_q[seg_last + 1];
  const int qlo_max = a.cu_q[seg_last], qhi_min = a.cu_q[seg_first + 1];

  const bf16x8 kf = row_frag(a.k, kc, H, head, half);
  const bf16x8 vf = row_frag(a.v, kc, H, head, half);
  int2 kn = make_int2(0, 0);
  int4 kmeta = make_int4(0, 0, 0, 0);
  if (MASKED) { kn = a.nodes[kc]; kmeta = a.meta[kt]; }
  const bf16x8 zfill = splat8(0.f);
  const f32x16 zero = {};
  f32x16 dva = {}, dka = {};
  const float* lse2h = a.lse2 + (size_t)head * a.tq_pad;
  const float* dvech = a.dvec + (size_t)head * a.tq_pad;

  const int qt_beg = qbeg >> 5, qt_end = (qend + kTile - 1) >> 5;
  for (int qt = qt_beg; qt < qt_end; ++qt) {
    const int q0 = qt * kTile;
    if (MASKED) {
      if (!tiles_may_touch(a.meta[qt], kmeta)) continue;
    }
    const int qr = min(q0 + kperm(col), a.total_q - 1);
    const bf16x8 qfa = row_frag(a.q, qr, H, head, half);
    const f32x16 s = mfma32(qfa, kf, zero);
    const bf16x8 dofa = row_frag(a.dout, qr, H, head, half);
    const f32x16 dp = mfma32(dofa, vf, zero);
    // Per-row (query) statistics: rows r -> q0 + 16(r>>3) + 8h + (r&7).
    const f32x4* l2p0 = reinterpret_cast<const f32x4*>(lse2h + q0 + 8 * half);
    const f32x4* l2p1 = reinterpret_cast<const f32x4*>(lse2h + q0 + 16 + 8 * half);
    const f32x4* dvp0 = reinterpret_cast<const f32x4*>(dvech + q0 + 8 * half);
    const f32x4* dvp1 = reinterpret_cast<const f32x4*>(dvech + q0 + 16 + 8 * half);
    const f32x4 la = l2p0[0], lb = l2p0[1], lc = l2p1[0], ld = l2p1[1];
    const f32x4 da = dvp0[0], db = dvp0[1], dc = dvp1[0], dd = dvp1[1];
    float l2[16], dr[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      l2[i] = la[i]; l2[4 + i] = lb[i]; l2[8 + i] = lc[i]; l2[12 + i] = ld[i];
      dr[i] = da[i]; dr[4 + i] = db[i]; dr[8 + i] = dc[i]; dr[12 + i] = dd[i];
    }
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = fast_exp2(fmaf(s[r], a.c, -l2[r]));
    const bool full = !MASKED && q0 >= qlo_max && q0 + kTile <= qhi_min;
    if (!full) {
      int2 qn[16];
      if (MASKED) load_nodes16(a.nodes, q0, half, qn);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qq = row_token(q0, r, half);
        bool ok = qq >= qlo && qq < qhi;
        if (MASKED) ok = ok && qq != ki && node_adjacent(qn[r], kn);
        p[r] = ok ? p[r] : 0.f;
      }
    }
    bf16x8 p0, p1, s0, s1;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p0[e] = (bf16)p[e];
      p1[e] = (bf16)p[8 + e];
      s0[e] = (bf16)(p[e] * (dp[e] - dr[e]));
      s1[e] = (bf16)(p[8 + e] * (dp[8 + e] - dr[8 + e]));
    }
    const int ch = (q0 >> 3) + half;
    dva = mfma32(tt_frag(a.dot, ch, H, head, col, zfill), p0, dva);
    dva = mfma32(tt_frag(a.dot, ch + 2, H, head, col, zfill), p1, dva);
    dka = mfma32(tt_frag(a.qt, ch, H, head, col, zfill), s0, dka);
    dka = mfma32(tt_frag(a.qt, ch + 2, H, head, col, zfill), s1, dka);
  }
  if (!kvalid) return;
  store_rows8(a.dv + ((size_t)ki * H + head) * kHd, dva, 1.f, half);
  store_rows8(a.dk + ((size_t)ki * H + head) * kHd, dka, a.scale, half);
}

// x [total][H][16] -> xt [tpad/8][H][16][8], zero beyond `total`.
__global__ void tt_transpose_kernel(const bf16* __restrict__ x, int total, int heads, int tpad,
                                    bf16* __restrict__ xt) {
  const long n = (long)(tpad / 8) * heads * kHd;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int d = (int)(idx % kHd);
  const int h = (int)((idx / kHd) % heads);
  const int c = (int)(idx / ((long)kHd * heads));
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int t = c * 8 + i;
    r[i] = t < total ? x[((size_t)t * heads + h) * kHd + d] : (bf16)0.f;
  }
  *reinterpret_cast<bf16x8*>(xt + idx * 8) = r;
}

// lse2 = lse * log2(e) (+inf for rows with no admissible key, and padding),
// dvec = rowsum(dO * O) in fp32.
__global__ void bwd_prep_kernel(const bf16* __restrict__ dout, const bf16* __restrict__ out,
                                const float* __restrict__ lse, int total_q, int heads, int tq_pad,
                                float* __restrict__ lse2, float* __restrict__ dvec) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)heads * tq_pad) return;
  const int h = (int)(idx / tq_pad), t = (int)(idx % tq_pad);
  float l2 = INFINITY, dsum = 0.f;
  if (t < total_q) {
    const float l = lse[(size_t)h * total_q + t];
    l2 = l == -INFINITY ? INFINITY : l * kLog2e;
    const bf16x8* po = reinterpret_cast<const bf16x8*>(out + ((size_t)t * heads + h) * kHd);
    const bf16x8* pd = reinterpret_cast<const bf16x8*>(dout + ((size_t)t * heads + h) * kHd);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const bf16x8 o = po[j], g = pd[j];
#pragma unroll
      for (int e = 0; e < 8; ++e) dsum = fmaf((float)o[e], (float)g[e], dsum);
    }
  }
  lse2[idx] = l2;
  dvec[idx] = dsum;
}

__global__ void nodes_pack_kernel(const int* __restrict__ src, const int* __restrict__ dst, int total,
                                  int tpad, int2* __restrict__ nodes) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= tpad) return;
  nodes[t] = t < total ? make_int2(src[t], dst[t]) : make_int2(-1, -1);
}

// Per 32-token tile: min / max node id over both endpoints and a 64-bit
// signature of (node & 63).
__global__ void tile_meta_kernel(const int2* __restrict__ nodes, int total, int n_tiles,
                                 int4* __restrict__ meta) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_tiles) return;
  int lo = INT_MAX, hi = INT_MIN;
  unsigned long long sig = 0ull;
  for (int i = 0; i < kTile; ++i) {
    const int tok = t * kTile + i;
    if (tok >= total) break;
    const int2 n = nodes[tok];
    lo = min(lo, min(n.x, n.y));
    hi = max(hi, max(n.x, n.y));
    sig |= (1ull << (n.x & 63)) | (1ull << (n.y & 63));
  }
  meta[t] = make_int4(lo, hi, (int)(sig & 0xffffffffull), (int)(sig >> 32));
}

// Longest-first order of the outer tiles by the number of inner tiles they
// visit (counting sort, one block).
__global__ __launch_bounds__(1024) void plan_kernel(const int* __restrict__ cu_outer,
                                                    const int* __restrict__ cu_inner, int nseg,
                                                    int total_outer, int n_tiles, int* __restrict__ plan) {
  constexpr int NB = 1024;
  __shared__ int hist[NB];
  const int tid = threadIdx.x;
  for (int i = tid; i < NB; i += blockDim.x) hist[i] = 0;
  __syncthreads();
  auto bucket = [&](int t) {
    const int o0 = t * kTile, o1 = min(o0 + kTile - 1, total_outer - 1);
    const int s0 = seg_of(cu_outer, nseg, o0), s1 = seg_of(cu_outer, nseg, o1);
    const int ib = cu_inner[s0], ie = cu_inner[s1 + 1];
    const int cost = ie > ib ? ((ie + kTile - 1) >> 5) - (ib >> 5) : 0;
    return NB - 1 - min(cost, NB - 1);
  };
  for (int t = tid; t < n_tiles; t += blockDim.x) atomicAdd(&hist[bucket(t)], 1);
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int i = 0; i < NB; ++i) { const int h = hist[i]; hist[i] = run; run += h; }
  }
  __syncthreads();
  for (int t = tid; t < n_tiles; t += blockDim.x) plan[atomicAdd(&hist[bucket(t)], 1)] = t;
}

__global__ void edge_mask_dense_kernel(const int* __restrict__ src, const int* __restrict__ dst,
                                       const int* __restrict__ cu, int batch, int max_items,
                                       uint8_t* __restrict__ mask) {
  const long n = (long)batch * max_items * max_items;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int j = (int)(idx % max_items);
  const int i = (int)((idx / max_items) % max_items);
  const int b = (int)(idx / ((long)max_items * max_items));
  const int start = cu[b], len = cu[b + 1] - start;
  uint8_t m = 0;
  if (i < len && j < len && i != j) {
    const int2 a = make_int2(src[start + i], dst[start + i]);
    const int2 c = make_int2(src[start + j], dst[start + j]);
    m = node_adjacent(a, c) ? 1 : 0;
  }
  mask[idx] = m;
}

// ---------------------------------------------------------------- host side

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
int round32(int x) { return (x + kTile - 1) / kTile * kTile; }

struct WsLayout {
  size_t vt = 0, qt = 0, kt = 0, dot = 0, lse2 = 0, dvec = 0, plan_q = 0, plan_k = 0,
         nodes = 0, meta = 0, total = 0;
};

WsLayout ws_layout(int total_q, int total_k, int heads, bool masked, bool backward) {
  WsLayout L;
  const int tqp = round32(total_q), tkp = round32(total_k);
  const size_t ttq = (size_t)tqp * heads * kHd * 2, ttk = (size_t)tkp * heads * kHd * 2;
  size_t off = 0;
  if (!backward) {
    L.vt = off; off += align256(ttk);
  } else {
    L.qt = off; off += align256(ttq);
    L.kt = off; off += align256(ttk);
    L.dot = off; off += align256(ttq);
    L.lse2 = off; off += align256((size_t)heads * tqp * 4);
    L.dvec = off; off += align256((size_t)heads * tqp * 4);
  }
  L.plan_q = off; off += align256((size_t)(tqp / kTile) * 4);
  if (backward) { L.plan_k = off; off += align256((size_t)(tkp / kTile) * 4); }
  if (masked) {
    L.nodes = off; off += align256((size_t)tqp * 8);
    L.meta = off; off += align256((size_t)(tqp / kTile) * 16);
  }
  L.total = off;
  return L;
}

bool misaligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; }

int check_common(int batch, int total_q, int total_k, int heads, int head_dim, bool masked) {
  if (head_dim != kHd) return ESA_ERR_HEAD_DIM;
  if (batch < 1 || heads < 1 || total_q < 0 || total_k < 0) return ESA_ERR_SHAPE;
  if ((long)total_q * heads * kHd >= (1L << 31) || (long)total_k * heads * kHd >= (1L << 31)) return ESA_ERR_SHAPE;
  if (masked && total_q != total_k) return ESA_ERR_MASK;
  return ESA_OK;
}

__global__ void zero16_kernel(uint4* __restrict__ p, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// Zero `bytes` (a multiple of 16) at a 16-byte aligned pointer.
int launch_zero(void* p, size_t bytes, hipStream_t st) {
  const long n = (long)(bytes / 16);
  if (n == 0) return ESA_OK;
  long g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  hipLaunchKernelGGL(zero16_kernel, dim3((unsigned)g), dim3(256), 0, st, static_cast<uint4*>(p), n);
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

int launch_tt(const bf16* x, int total, int heads, bf16* xt, hipStream_t st) {
  const int tp = round32(total);
  const long n = (long)(tp / 8) * heads * kHd;
  if (n == 0) return ESA_OK;
  ESA_TIMED(esa_profile::kAttnPrep, st,
            hipLaunchKernelGGL(tt_transpose_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, total,
                               heads, tp, xt));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

int launch_mask_meta(const int* src, const int* dst, int total, int2* nodes, int4* meta, hipStream_t st) {
  const int tp = round32(total);
  ESA_TIMED(esa_profile::kAttnPrep, st,
            hipLaunchKernelGGL(nodes_pack_kernel, dim3((unsigned)((tp + 255) / 256)), dim3(256), 0, st, src, dst,
                               total, tp, nodes));
  ESA_LAUNCH_CHECK();
  const int nt = tp / kTile;
  ESA_TIMED(esa_profile::kAttnPrep, st,
            hipLaunchKernelGGL(tile_meta_kernel, dim3((unsigned)((nt + 255) / 256)), dim3(256), 0, st, nodes, total,
                               nt, meta));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

int launch_plan(const int* cu_outer, const int* cu_inner, int nseg, int total_outer, int* plan, hipStream_t st) {
  const int nt = round32(total_outer) / kTile;
  ESA_TIMED(esa_profile::kAttnPrep, st,
            hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(1024), 0, st, cu_outer, cu_inner, nseg, total_outer, nt,
                               plan));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

}  // namespace

extern "C" {

const char* esa_version(void) { return "esa_hip 0.1 gfx950"; }

int esa_varlen_attn_workspace_size(int total_q, int total_k, int heads, int head_dim, int masked,
                                   int backward, size_t* bytes) {
  if (!bytes) return ESA_ERR_NULL;
  const int rc = check_common(1, total_q, total_k, heads, head_dim, masked != 0);
  if (rc) return rc;
  *bytes = ws_layout(total_q, total_k, heads, masked != 0, backward != 0).total;
  return ESA_OK;
}

int esa_varlen_attn_fwd(const void* q, const void* k, const void* v, const int* cu_seqlens_q,
                        const int* cu_seqlens_k, int batch, int total_q, int total_k,
                        int max_seqlen_q, int max_seqlen_k, int heads, int head_dim,
                        float softmax_scale, const int* tok_src, const int* tok_dst, void* out,
                        float* softmax_lse, void* workspace, size_t workspace_bytes, void* stream) {
  (void)max_seqlen_q; (void)max_seqlen_k;
  const bool masked = tok_src != nullptr || tok_dst != nullptr;
  if (masked && (!tok_src || !tok_dst)) return ESA_ERR_NULL;
  int rc = check_common(batch, total_q, total_k, heads, head_dim, masked);
  if (rc) return rc;
  if (total_q == 0) return ESA_OK;
  if (!q || !k || !v || !cu_seqlens_q || !cu_seqlens_k || !out || !softmax_lse || !workspace) return ESA_ERR_NULL;
  if (misaligned(q) || misaligned(k) || misaligned(v) || misaligned(out) || misaligned(workspace)) return ESA_ERR_ALIGN;
  const WsLayout L = ws_layout(total_q, total_k, heads, masked, false);
  if (workspace_bytes < L.total) return ESA_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);

  QOuterArgs a{};
  a.q = static_cast<const bf16*>(q); a.k = static_cast<const bf16*>(k); a.v = static_cast<const bf16*>(v);
  a.at = reinterpret_cast<const bf16*>(ws + L.vt);
  a.cu_q = cu_seqlens_q; a.cu_k = cu_seqlens_k; a.nseg = batch;
  a.total_q = total_q; a.total_k = total_k; a.heads = heads; a.tq_pad = round32(total_q);
  a.scale = softmax_scale; a.c = softmax_scale * kLog2e;
  a.plan = reinterpret_cast<const int*>(ws + L.plan_q);
  a.n_tiles = round32(total_q) / kTile;
  a.out = static_cast<bf16*>(out); a.lse = softmax_lse;
  if (total_k > 0) {
    if ((rc = launch_tt(a.v, total_k, heads, reinterpret_cast<bf16*>(ws + L.vt), st))) return rc;
  }
  if (masked) {
    a.nodes = reinterpret_cast<const int2*>(ws + L.nodes);
    a.meta = reinterpret_cast<const int4*>(ws + L.meta);
    if ((rc = launch_mask_meta(tok_src, tok_dst, total_q, reinterpret_cast<int2*>(ws + L.nodes),
                               reinterpret_cast<int4*>(ws + L.meta), st))) return rc;
  }
  if ((rc = launch_plan(cu_seqlens_q, cu_seqlens_k, batch, total_q, reinterpret_cast<int*>(ws + L.plan_q), st))) return rc;
  const unsigned grid = (unsigned)a.n_tiles * (unsigned)((heads + 3) / 4);
  if (masked)
    ESA_TIMED(esa_profile::kAttnFwdMasked, st,
              hipLaunchKernelGGL((attn_qouter_kernel<true, false>), dim3(grid), dim3(256), 0, st, a));
  else
    ESA_TIMED(esa_profile::kAttnFwd, st,
              hipLaunchKernelGGL((attn_qouter_kernel<false, false>), dim3(grid), dim3(256), 0, st, a));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

int esa_varlen_attn_bwd(const void* dout, const void* q, const void* k, const void* v, const void* out,
                        const float* softmax_lse, const int* cu_seqlens_q, const int* cu_seqlens_k,
                        int batch, int total_q, int total_k, int max_seqlen_q, int max_seqlen_k,
                        int heads, int head_dim, float softmax_scale, const int* tok_src,
                        const int* tok_dst, void* dq, void* dk, void* dv, void* workspace,
                        size_t workspace_bytes, void* stream) {
  (void)max_seqlen_q; (void)max_seqlen_k;
  const bool masked = tok_src != nullptr || tok_dst != nullptr;
  if (masked && (!tok_src || !tok_dst)) return ESA_ERR_NULL;
  int rc = check_common(batch, total_q, total_k, heads, head_dim, masked);
  if (rc) return rc;
  if (!dout || !q || !k || !v || !out || !softmax_lse || !cu_seqlens_q || !cu_seqlens_k || !dq || !dk ||
      !dv || !workspace)
    return ESA_ERR_NULL;
  if (misaligned(dout) || misaligned(q) || misaligned(k) || misaligned(v) || misaligned(out) ||
      misaligned(dq) || misaligned(dk) || misaligned(dv) || misaligned(workspace))
    return ESA_ERR_ALIGN;
  const WsLayout L = ws_layout(total_q, total_k, heads, masked, true);
  if (workspace_bytes < L.total) return ESA_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  if (total_q == 0 || total_k == 0) {
    // No query/key pairs: every gradient is zero (a fill kernel, so the call
    // stays capturable in a HIP graph).
    if ((rc = launch_zero(dq, (size_t)total_q * heads * kHd * 2, st))) return rc;
    if ((rc = launch_zero(dk, (size_t)total_k * heads * kHd * 2, st))) return rc;
    if ((rc = launch_zero(dv, (size_t)total_k * heads * kHd * 2, st))) return rc;
    return ESA_OK;
  }
  const int tqp = round32(total_q);
  bf16* qt = reinterpret_cast<bf16*>(ws + L.qt);
  bf16* ktt = reinterpret_cast<bf16*>(ws + L.kt);
  bf16* dot = reinterpret_cast<bf16*>(ws + L.dot);
  float* lse2 = reinterpret_cast<float*>(ws + L.lse2);
  float* dvec = reinterpret_cast<float*>(ws + L.dvec);
  int* plan_q = reinterpret_cast<int*>(ws + L.plan_q);
  int* plan_k = reinterpret_cast<int*>(ws + L.plan_k);
  if ((rc = launch_tt(static_cast<const bf16*>(q), total_q, heads, qt, st))) return rc;
  if ((rc = launch_tt(static_cast<const bf16*>(k), total_k, heads, ktt, st))) return rc;
  if ((rc = launch_tt(static_cast<const bf16*>(dout), total_q, heads, dot, st))) return rc;
  {
    const long n = (long)heads * tqp;
    ESA_TIMED(esa_profile::kAttnPrep, st,
              hipLaunchKernelGGL(bwd_prep_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                                 static_cast<const bf16*>(dout), static_cast<const bf16*>(out), softmax_lse,
                                 total_q, heads, tqp, lse2, dvec));
    ESA_LAUNCH_CHECK();
  }
  const int2* nodes = nullptr;
  const int4* meta = nullptr;
  if (masked) {
    nodes = reinterpret_cast<const int2*>(ws + L.nodes);
    meta = reinterpret_cast<const int4*>(ws + L.meta);
    if ((rc = launch_mask_meta(tok_src, tok_dst, total_q, reinterpret_cast<int2*>(ws + L.nodes),
                               reinterpret_cast<int4*>(ws + L.meta), st))) return rc;
  }
  if ((rc = launch_plan(cu_seqlens_q, cu_seqlens_k, batch, total_q, plan_q, st))) return rc;
  if ((rc = launch_plan(cu_seqlens_k, cu_seqlens_q, batch, total_k, plan_k, st))) return rc;
  const float c = softmax_scale * kLog2e;
  const unsigned groups = (unsigned)((heads + 3) / 4);

  KOuterArgs ka{};
  ka.q = static_cast<const bf16*>(q); ka.k = static_cast<const bf16*>(k); ka.v = static_cast<const bf16*>(v);
  ka.dout = static_cast<const bf16*>(dout); ka.qt = qt; ka.dot = dot; ka.lse2 = lse2; ka.dvec = dvec;
  ka.cu_q = cu_seqlens_q; ka.cu_k = cu_seqlens_k; ka.nseg = batch;
  ka.total_q = total_q; ka.total_k = total_k; ka.heads = heads; ka.tq_pad = tqp;
  ka.c = c; ka.scale = softmax_scale; ka.nodes = nodes; ka.meta = meta;
  ka.plan = plan_k; ka.n_tiles = round32(total_k) / kTile;
  ka.dk = static_cast<bf16*>(dk); ka.dv = static_cast<bf16*>(dv);
  const unsigned kgrid = (unsigned)ka.n_tiles * groups;
  if (masked)
    ESA_TIMED(esa_profile::kAttnBwdDkdvMasked, st,
              hipLaunchKernelGGL((attn_kouter_kernel<true>), dim3(kgrid), dim3(256), 0, st, ka));
  else
    ESA_TIMED(esa_profile::kAttnBwdDkdv, st,
              hipLaunchKernelGGL((attn_kouter_kernel<false>), dim3(kgrid), dim3(256), 0, st, ka));
  ESA_LAUNCH_CHECK();

  QOuterArgs qa{};
  qa.q = ka.q; qa.k = ka.k; qa.v = ka.v; qa.at = ktt; qa.dout = ka.dout; qa.lse2 = lse2; qa.dvec = dvec;
  qa.cu_q = cu_seqlens_q; qa.cu_k = cu_seqlens_k; qa.nseg = batch;
  qa.total_q = total_q; qa.total_k = total_k; qa.heads = heads; qa.tq_pad = tqp;
  qa.c = c; qa.scale = softmax_scale; qa.nodes = nodes; qa.meta = meta;
  qa.plan = plan_q; qa.n_tiles = tqp / kTile; qa.dq = static_cast<bf16*>(dq);
  const unsigned qgrid = (unsigned)qa.n_tiles * groups;
  if (masked)
    ESA_TIMED(esa_profile::kAttnBwdDqMasked, st,
              hipLaunchKernelGGL((attn_qouter_kernel<true, true>), dim3(qgrid), dim3(256), 0, st, qa));
  else
    ESA_TIMED(esa_profile::kAttnBwdDq, st,
              hipLaunchKernelGGL((attn_qouter_kernel<false, true>), dim3(qgrid), dim3(256), 0, st, qa));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

int esa_edge_mask_dense(const int* tok_src, const int* tok_dst, const int* cu_seqlens, int batch, int total,
                        int max_items, uint8_t* mask_out, void* stream) {
  (void)total;
  if (!tok_src || !tok_dst || !cu_seqlens || !mask_out) return ESA_ERR_NULL;
  if (batch < 1 || max_items < 0) return ESA_ERR_SHAPE;
  const long n = (long)batch * max_items * max_items;
  if (n == 0) return ESA_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(edge_mask_dense_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, tok_src, tok_dst,
                     cu_seqlens, batch, max_items, mask_out);
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

}  // extern "C"
