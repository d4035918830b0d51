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
//   stay per lane (one query per lane).
//   V^T (and K^T, Q^T, dO^T in backward) is pre-transposed into a
//   tile-transposed layout [T/8][H][rows][8] so each lane's A operand is one
//   aligned 16-byte load; the forward's V^T carries the ones as rows 16..31.
//
// Softmax reference point.  By Cauchy-Schwarz every score of query i obeys
// c*|S_ij| <= c*|q_i|*max_j|k_j| =: b_i (c = scale*log2 e).  When b_i <= 60 for
// every query of a wave, exp2(c*S_ij - b_i) lies in [2^-120, 1]: no overflow,
// no underflow, so softmax(S) = p / sum(p) with the fixed reference b_i is
// exact up to rounding and needs no running max and no rescaling.  Waves with
// a larger bound take the online (running-max) path.
//
// Loads go through buffer resources with the tensor's byte size as range:
// the hardware returns 0 for any part of a load past the end, so tiles that
// run past the last token need no index clamping.
#include "esa_common.h"
#include "esa_profile.h"
#include "../../include/esa_hip.h"

namespace {

constexpr int kTile = 32;
constexpr int kHd = 16;
constexpr float kStaticBound = 60.f;

typedef __amdgpu_buffer_rsrc_t rsrc_t;

DEVI rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
DEVI bf16x8 bload16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

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

struct QOuterArgs {
  const bf16* q; const bf16* k; const bf16* v;
  const bf16* at;          // forward: V^T with ones rows [Tk/8][H][32][8]; dQ pass: K^T [Tk/8][H][16][8]
  uint32_t at_bytes;
  const bf16* dout;        // dQ pass
  const float* lse2;       // dQ pass: log2-domain LSE [H][tq_pad], +inf = row without keys
  const float* dvec;       // dQ pass: rowsum(dO * O) [H][tq_pad]
  const float* knorm;      // forward: max |k| per (head, key tile) [H][tk_tiles]
  const int* cu_q; const int* cu_k; int nseg;
  int total_q, total_k, heads, tq_pad, tk_tiles;
  float c;                 // softmax_scale * log2(e)
  float scale;
  const int2* nodes; const int4* meta;
  const int* plan; int n_tiles;
  bf16* out; float* lse;   // forward outputs
  bf16* dq;                // dQ pass output
};

// Per-wave state of a Q-outer pass.
struct QWave {
  int col, half, qi, klo, khi, klo_max, khi_min, kt_beg, kt_end;
  bf16x8 qf;
  int2 qn;
  int4 qmeta;
};

// Score tile S^T for key tile kt (K fragment kf) with out-of-segment /
// masked entries at -inf.
template <bool MASKED>
DEVI f32x16 score_tile(const QOuterArgs& a, const QWave& w, const bf16x8& kf, int kt) {
  const f32x16 zero = {};
  f32x16 s = mfma32(kf, w.qf, zero);
  const int k0 = kt * kTile;
  const bool full = !MASKED && k0 >= w.klo_max && k0 + kTile <= w.khi_min;
  if (!full) {
    int2 kn[16];
    if (MASKED) load_nodes16(a.nodes, k0, w.half, kn);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = row_token(k0, r, w.half);
      bool ok = key >= w.klo && key < w.khi;
      if (MASKED) ok = ok && key != w.qi && node_adjacent(kn[r], w.qn);
      s[r] = ok ? s[r] : -INFINITY;
    }
  }
  return s;
}

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
  QWave w;
  w.col = lane & 31;
  w.half = lane >> 5;
  const int col = w.col, half = w.half;
  w.qi = q0 + col;
  const bool qvalid = w.qi < a.total_q;
  const int qc = qvalid ? w.qi : a.total_q - 1;
  const int q_last = min(q0 + kTile - 1, a.total_q - 1);
  const int seg_first = seg_of(a.cu_q, a.nseg, q0);
  const int seg_last = seg_of(a.cu_q, a.nseg, q_last);
  const int seg = seg_of(a.cu_q, a.nseg, qc);
  w.klo = qvalid ? a.cu_k[seg] : 0;
  w.khi = qvalid ? a.cu_k[seg + 1] : 0;
  const int kbeg = a.cu_k[seg_first], kend = a.cu_k[seg_last + 1];
  w.klo_max = a.cu_k[seg_last];
  w.khi_min = a.cu_k[seg_first + 1];
  w.kt_beg = kbeg >> 5;
  w.kt_end = (kend + kTile - 1) >> 5;
  w.qf = *reinterpret_cast<const bf16x8*>(a.q + ((size_t)qc * H + head) * kHd + 8 * half);
  w.qn = make_int2(0, 0);
  w.qmeta = make_int4(0, 0, 0, 0);
  if (MASKED) { w.qn = a.nodes[qc]; w.qmeta = a.meta[qt]; }

  const rsrc_t rk = make_rsrc(a.k, (uint32_t)a.total_k * H * kHd * 2);
  const rsrc_t ra = make_rsrc(a.at, a.at_bytes);
  constexpr int ROWS = DQ ? 16 : 32;
  const uint32_t k_step = (uint32_t)kTile * H * kHd * 2;
  const uint32_t chunk_bytes = (uint32_t)H * ROWS * 16;
  uint32_t koff = ((uint32_t)(w.kt_beg * kTile + kperm(col)) * H + head) * (kHd * 2) + 16u * half;
  uint32_t aoff = ((uint32_t)(w.kt_beg * 4 + half) * H * ROWS + head * ROWS + (DQ ? (col & 15) : col)) * 16u;
  const uint32_t a_step = 4u * chunk_bytes;

  f32x16 acc = {};
  if (!DQ) {
    // Reference point b = c |q| max|k| (see the file comment).
    float qq = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) qq = fmaf((float)w.qf[e], (float)w.qf[e], qq);
    qq += __shfl_xor(qq, 32);
    float km = 0.f;
    for (int t = w.kt_beg + lane; t < w.kt_end; t += 64) km = fmaxf(km, a.knorm[(size_t)head * a.tk_tiles + t]);
    km = wave_max(km);
    const float b = a.c * sqrtf(qq) * km;
    const bool fixed_ref = wave_max(qvalid ? b : 0.f) <= kStaticBound;
    float m_run;
    if (fixed_ref) {
      m_run = b;
      // Loads run one tile ahead (past the end they read zeros, unused).
      bf16x8 kf = bload16(rk, koff);
      for (int kt = w.kt_beg; kt < w.kt_end; ++kt) {
        if (MASKED && !tiles_may_touch(w.qmeta, a.meta[kt])) {
          koff += k_step; aoff += a_step;
          kf = bload16(rk, koff);
          continue;
        }
        const bf16x8 v0 = bload16(ra, aoff), v1 = bload16(ra, aoff + 2 * chunk_bytes);
        const f32x16 s = score_tile<MASKED>(a, w, kf, kt);
        koff += k_step; aoff += a_step;
        kf = bload16(rk, koff);
        float p[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = fast_exp2(fmaf(s[r], a.c, -b));
        acc = mfma32(v0, cvt8(p), acc);
        acc = mfma32(v1, cvt8(p + 8), acc);
      }
    } else {
      m_run = -INFINITY;
      for (int kt = w.kt_beg; kt < w.kt_end; ++kt, koff += k_step, aoff += a_step) {
        if (MASKED && !tiles_may_touch(w.qmeta, a.meta[kt])) continue;
        const f32x16 s = score_tile<MASKED>(a, w, bload16(rk, koff), kt);
        float mt = s[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float m_new = fmaxf(m_run, mt * a.c);
        if (__ballot(m_new > m_run)) {
          const float alpha = fast_exp2(m_run - (m_new == -INFINITY ? 0.f : m_new));
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[r] *= alpha;
          m_run = m_new;
        }
        const float m_use = m_run == -INFINITY ? 0.f : m_run;
        float p[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = fast_exp2(fmaf(s[r], a.c, -m_use));
        acc = mfma32(bload16(ra, aoff), cvt8(p), acc);
        acc = mfma32(bload16(ra, aoff + 2 * chunk_bytes), cvt8(p + 8), acc);
      }
    }
    if (!qvalid) return;
    const float l = acc[8];  // a ones row of [V^T; 1] P^T: the softmax row sum
    const float inv = l > 0.f ? 1.f / l : 0.f;
    store_rows8(a.out + ((size_t)w.qi * H + head) * kHd, acc, inv, half);
    if (half == 0)
      a.lse[(size_t)head * a.total_q + w.qi] = l > 0.f ? (m_run + fast_log2(l)) * kLn2 : -INFINITY;
  } else {
    const bf16x8 dof = *reinterpret_cast<const bf16x8*>(a.dout + ((size_t)qc * H + head) * kHd + 8 * half);
    const float lse2q = a.lse2[(size_t)head * a.tq_pad + qc];
    const float dq_d = a.dvec[(size_t)head * a.tq_pad + qc];
    const rsrc_t rv = make_rsrc(a.v, (uint32_t)a.total_k * H * kHd * 2);
    const f32x16 zero = {};
    // Loads run one tile ahead (past the end they read zeros, unused).
    bf16x8 kf = bload16(rk, koff), vf = bload16(rv, koff);
    for (int kt = w.kt_beg; kt < w.kt_end; ++kt) {
      if (MASKED && !tiles_may_touch(w.qmeta, a.meta[kt])) {
        koff += k_step; aoff += a_step;
        kf = bload16(rk, koff); vf = bload16(rv, koff);
        continue;
      }
      const bf16x8 t0 = bload16(ra, aoff), t1 = bload16(ra, aoff + 2 * chunk_bytes);
      const f32x16 s = score_tile<MASKED>(a, w, kf, kt);
      const f32x16 dp = mfma32(vf, dof, zero);   // dP^T = V dO^T (V rows in K's order)
      koff += k_step; aoff += a_step;
      kf = bload16(rk, koff); vf = bload16(rv, koff);
      float ds[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) ds[r] = fast_exp2(fmaf(s[r], a.c, -lse2q)) * (dp[r] - dq_d);
      acc = mfma32(t0, cvt8(ds), acc);
      acc = mfma32(t1, cvt8(ds + 8), acc);
    }
    if (!qvalid) return;
    store_rows8(a.dq + ((size_t)w.qi * H + head) * kHd, acc, a.scale, half);
  }
}

struct KOuterArgs {
  const bf16* q; const bf16* k; const bf16* v; const bf16* dout;
  const bf16* qt; const bf16* dot;   // tile-transposed Q and dO [Tq/8][H][16][8]
  uint32_t tt_bytes;
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
  const int qlo = kvalid ? a.cu_q[seg] : 0, qhi = kvalid ? a.cu_q[seg + 1] : 0;
  const int qbeg = a.cu_q[seg_first], qend = a.cu_q[seg_last + 1];
  const int qlo_max = a.cu_q[seg_last], qhi_min = a.cu_q[seg_first + 1];

  const bf16x8 kf = *reinterpret_cast<const bf16x8*>(a.k + ((size_t)kc * H + head) * kHd + 8 * half);
  const bf16x8 vf = *reinterpret_cast<const bf16x8*>(a.v + ((size_t)kc * H + head) * kHd + 8 * half);
  int2 kn = make_int2(0, 0);
  int4 kmeta = make_int4(0, 0, 0, 0);
  if (MASKED) { kn = a.nodes[kc]; kmeta = a.meta[kt]; }
  const f32x16 zero = {};
  f32x16 dva = {}, dka = {};
  const float* lse2h = a.lse2 + (size_t)head * a.tq_pad + 8 * half;
  const float* dvech = a.dvec + (size_t)head * a.tq_pad + 8 * half;

  const rsrc_t rq = make_rsrc(a.q, (uint32_t)a.total_q * H * kHd * 2);
  const rsrc_t rdo = make_rsrc(a.dout, (uint32_t)a.total_q * H * kHd * 2);
  const rsrc_t rqt = make_rsrc(a.qt, a.tt_bytes);
  const rsrc_t rdot = make_rsrc(a.dot, a.tt_bytes);
  const int qt_beg = qbeg >> 5, qt_end = (qend + kTile - 1) >> 5;
  const uint32_t q_step = (uint32_t)kTile * H * kHd * 2;
  const uint32_t chunk_bytes = (uint32_t)H * 16 * 16;
  uint32_t qoff = ((uint32_t)(qt_beg * kTile + kperm(col)) * H + head) * (kHd * 2) + 16u * half;
  uint32_t toff = ((uint32_t)(qt_beg * 4 + half) * H * 16 + head * 16 + (col & 15)) * 16u;

  // Row fragments run one tile ahead (past the end they read zeros, unused).
  bf16x8 qa = bload16(rq, qoff), da = bload16(rdo, qoff);
  for (int qt = qt_beg; qt < qt_end; ++qt) {
    const int q0 = qt * kTile;
    if (MASKED && !tiles_may_touch(a.meta[qt], kmeta)) {
      qoff += q_step; toff += 4 * chunk_bytes;
      qa = bload16(rq, qoff); da = bload16(rdo, qoff);
      continue;
    }
    const bf16x8 o0 = bload16(rdot, toff), o1 = bload16(rdot, toff + 2 * chunk_bytes);
    const bf16x8 t0 = bload16(rqt, toff), t1 = bload16(rqt, toff + 2 * chunk_bytes);
    const f32x16 s = mfma32(qa, kf, zero);     // S = Q K^T, lane = key
    const f32x16 dp = mfma32(da, vf, zero);    // dP = dO V^T
    qoff += q_step; toff += 4 * chunk_bytes;
    qa = bload16(rq, qoff); da = bload16(rdo, qoff);
    // Per-row (query) statistics: rows r -> q0 + 16(r>>3) + 8h + (r&7).
    const f32x4* l2p = reinterpret_cast<const f32x4*>(lse2h + q0);
    const f32x4* dvp = reinterpret_cast<const f32x4*>(dvech + q0);
    const f32x4 la = l2p[0], lb = l2p[1], lc = l2p[4], ld = l2p[5];
    const f32x4 da = dvp[0], db = dvp[1], dc = dvp[4], dd = dvp[5];
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
    float ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) ds[r] = p[r] * (dp[r] - dr[r]);
    dva = mfma32(o0, cvt8(p), dva);
    dva = mfma32(o1, cvt8(p + 8), dva);
    dka = mfma32(t0, cvt8(ds), dka);
    dka = mfma32(t1, cvt8(ds + 8), dka);
  }
  if (!kvalid) return;
  store_rows8(a.dv + ((size_t)ki * H + head) * kHd, dva, 1.f, half);
  store_rows8(a.dk + ((size_t)ki * H + head) * kHd, dka, a.scale, half);
}

// ------------------------------------------------------------------ prep kernels

// One block per 32-token tile of x [total][H][16].
//  - xt != null: writes the tile-transposed layout [T/8][H][rows][8] for the
//    tile's four 8-token chunks: rows 0..15 are x's feature dims (zero past
//    `total`); rows 16..31 (rows == 32) are ones.
//  - knorm != null: writes max over the tile's tokens of |x_t| per head to
//    knorm[h * n_tiles + tile].
__global__ __launch_bounds__(256) void tile_transpose_kernel(const bf16* __restrict__ x, int total, int heads,
                                                             int rows, bf16* __restrict__ xt,
                                                             float* __restrict__ knorm, int n_tiles) {
  const int tile = blockIdx.x;
  const int t0 = tile * kTile;
  if (xt) {
    const int items = 4 * heads * rows;
    for (int it = threadIdx.x; it < items; it += blockDim.x) {
      const int r = it % rows;
      const int h = (it / rows) % heads;
      const int c = it / (rows * heads);
      bf16x8 o;
      if (r < kHd) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int t = t0 + c * 8 + i;
          o[i] = t < total ? x[((size_t)t * heads + h) * kHd + r] : (bf16)0.f;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (bf16)1.f;
      }
      *reinterpret_cast<bf16x8*>(xt + (((size_t)(tile * 4 + c) * heads + h) * rows + r) * 8) = o;
    }
  }
  if (knorm) {
    // one thread per head: max over the tile's tokens of the squared norm
    for (int h = threadIdx.x; h < heads; h += blockDim.x) {
      float m = 0.f;
      for (int i = 0; i < kTile && t0 + i < total; ++i) {
        const bf16x8* p = reinterpret_cast<const bf16x8*>(x + ((size_t)(t0 + i) * heads + h) * kHd);
        const bf16x8 u = p[0], v = p[1];
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) s = fmaf((float)u[e], (float)u[e], fmaf((float)v[e], (float)v[e], s));
        m = fmaxf(m, s);
      }
      knorm[(size_t)h * n_tiles + tile] = sqrtf(m);
    }
  }
}

// lse2 = lse * log2(e) (+inf for rows with no admissible key, and padding),
// dvec = rowsum(dO * O) in fp32.  Thread per (token, head), head fastest.
__global__ void bwd_rowstats_kernel(const bf16* __restrict__ dout, const bf16* __restrict__ out,
                                    const float* __restrict__ lse, int total_q, int heads, int tq_pad,
                                    float* __restrict__ lse2, float* __restrict__ dvec) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)heads * tq_pad) return;
  const int h = (int)(idx % heads), t = (int)(idx / heads);
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
  lse2[(size_t)h * tq_pad + t] = l2;
  dvec[(size_t)h * tq_pad + t] = dsum;
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
// visit (counting sort in one block; parallel scan of the bucket counts).
__global__ __launch_bounds__(1024) void plan_kernel(const int* __restrict__ cu_outer,
                                                    const int* __restrict__ cu_inner, int nseg,
                                                    int total_outer, int n_tiles, int* __restrict__ plan) {
  constexpr int NB = 1024;
  __shared__ int hist[NB];
  const int tid = threadIdx.x;
  hist[tid] = 0;
  __syncthreads();
  auto bucket = [&](int t) {
    const int o0 = t * kTile, o1 = min(o0 + kTile - 1, total_outer - 1);
    const int s0 = seg_of(cu_outer, nseg, o0), s1 = seg_of(cu_outer, nseg, o1);
    const int ib = cu_inner[s0], ie = cu_inner[s1 + 1];
    const int cost = ie > ib ? ((ie + kTile - 1) >> 5) - (ib >> 5) : 0;
    return NB - 1 - min(cost, NB - 1);
  };
  for (int t = tid; t < n_tiles; t += NB) atomicAdd(&hist[bucket(t)], 1);
  __syncthreads();
  // inclusive Hillis-Steele scan over the buckets, then shift to exclusive
  const int own = hist[tid];
  for (int off = 1; off < NB; off <<= 1) {
    const int add = tid >= off ? hist[tid - off] : 0;
    __syncthreads();
    hist[tid] += add;
    __syncthreads();
  }
  hist[tid] -= own;
  __syncthreads();
  for (int t = tid; t < n_tiles; t += NB) plan[atomicAdd(&hist[bucket(t)], 1)] = t;
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
    const int2 x = make_int2(src[start + i], dst[start + i]);
    const int2 y = make_int2(src[start + j], dst[start + j]);
    m = node_adjacent(x, y) ? 1 : 0;
  }
  mask[idx] = m;
}

__global__ void zero16_kernel(uint4* __restrict__ p, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// ---------------------------------------------------------------- host side

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
int round32(int x) { return (x + kTile - 1) / kTile * kTile; }

struct WsLayout {
  size_t vt = 0, knorm = 0, qt = 0, kt = 0, dot = 0, lse2 = 0, dvec = 0, plan_q = 0, plan_k = 0,
         nodes = 0, meta = 0, total = 0;
  size_t vt_bytes = 0, tt_q_bytes = 0, tt_k_bytes = 0;
};

WsLayout ws_layout(int total_q, int total_k, int heads, bool masked, bool backward) {
  WsLayout L;
  const int tqp = round32(total_q), tkp = round32(total_k);
  size_t off = 0;
  if (!backward) {
    L.vt_bytes = (size_t)tkp * heads * 32 * 2;
    L.vt = off; off += align256(L.vt_bytes);
    L.knorm = off; off += align256((size_t)heads * (tkp / kTile) * 4);
  } else {
    L.tt_q_bytes = (size_t)tqp * heads * kHd * 2;
    L.tt_k_bytes = (size_t)tkp * heads * kHd * 2;
    L.qt = off; off += align256(L.tt_q_bytes);
    L.kt = off; off += align256(L.tt_k_bytes);
    L.dot = off; off += align256(L.tt_q_bytes);
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
  // Buffer-resource ranges are 32-bit byte counts; the forward's V^T has 32 rows per head.
  const long lim = (1L << 31) - 1;
  if ((long)round32(total_q) * heads * 64 > lim || (long)round32(total_k) * heads * 64 > lim) return ESA_ERR_SHAPE;
  if (masked && total_q != total_k) return ESA_ERR_MASK;
  return ESA_OK;
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

int launch_tt(const bf16* x, int total, int heads, int rows, bf16* xt, float* knorm, hipStream_t st) {
  const int nt = round32(total) / kTile;
  if (nt == 0) return ESA_OK;
  ESA_TIMED(esa_profile::kAttnPrep, st,
            hipLaunchKernelGGL(tile_transpose_kernel, dim3((unsigned)nt), dim3(256), 0, st, x, total, heads, rows,
                               xt, knorm, nt));
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

const char* esa_version(void) { return "esa_hip 0.2 gfx950"; }

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
  if (!(softmax_scale > 0.f)) return ESA_ERR_SHAPE;
  const WsLayout L = ws_layout(total_q, total_k, heads, masked, false);
  if (workspace_bytes < L.total) return ESA_ERR_WORKSPACE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);

  QOuterArgs a{};
  a.q = static_cast<const bf16*>(q); a.k = static_cast<const bf16*>(k); a.v = static_cast<const bf16*>(v);
  a.at = reinterpret_cast<const bf16*>(ws + L.vt);
  a.at_bytes = (uint32_t)L.vt_bytes;
  a.knorm = reinterpret_cast<const float*>(ws + L.knorm);
  a.cu_q = cu_seqlens_q; a.cu_k = cu_seqlens_k; a.nseg = batch;
  a.total_q = total_q; a.total_k = total_k; a.heads = heads; a.tq_pad = round32(total_q);
  a.tk_tiles = round32(total_k) / kTile;
  a.scale = softmax_scale; a.c = softmax_scale * kLog2e;
  a.plan = reinterpret_cast<const int*>(ws + L.plan_q);
  a.n_tiles = round32(total_q) / kTile;
  a.out = static_cast<bf16*>(out); a.lse = softmax_lse;
  if (total_k > 0) {
    if ((rc = launch_tt(a.v, total_k, heads, 32, reinterpret_cast<bf16*>(ws + L.vt), nullptr, st))) return rc;
    if ((rc = launch_tt(a.k, total_k, heads, 0, nullptr, reinterpret_cast<float*>(ws + L.knorm), st))) return rc;
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
  if (total_q == 0 && total_k == 0) return ESA_OK;
  if (!dout || !q || !k || !v || !out || !softmax_lse || !cu_seqlens_q || !cu_seqlens_k || !dq || !dk ||
      !dv || !workspace)
    return ESA_ERR_NULL;
  if (misaligned(dout) || misaligned(q) || misaligned(k) || misaligned(v) || misaligned(out) ||
      misaligned(dq) || misaligned(dk) || misaligned(dv) || misaligned(workspace))
    return ESA_ERR_ALIGN;
  if (!(softmax_scale > 0.f)) return ESA_ERR_SHAPE;
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
  if ((rc = launch_tt(static_cast<const bf16*>(q), total_q, heads, 16, qt, nullptr, st))) return rc;
  if ((rc = launch_tt(static_cast<const bf16*>(k), total_k, heads, 16, ktt, nullptr, st))) return rc;
  if ((rc = launch_tt(static_cast<const bf16*>(dout), total_q, heads, 16, dot, nullptr, st))) return rc;
  {
    const long n = (long)heads * tqp;
    ESA_TIMED(esa_profile::kAttnPrep, st,
              hipLaunchKernelGGL(bwd_rowstats_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
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
  ka.dout = static_cast<const bf16*>(dout); ka.qt = qt; ka.dot = dot; ka.tt_bytes = (uint32_t)L.tt_q_bytes;
  ka.lse2 = lse2; ka.dvec = dvec;
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
  qa.q = ka.q; qa.k = ka.k; qa.v = ka.v; qa.at = ktt; qa.at_bytes = (uint32_t)L.tt_k_bytes;
  qa.dout = ka.dout; qa.lse2 = lse2; qa.dvec = dvec;
  qa.cu_q = cu_seqlens_q; qa.cu_k = cu_seqlens_k; qa.nseg = batch;
  qa.total_q = total_q; qa.total_k = total_k; qa.heads = heads; qa.tq_pad = tqp;
  qa.tk_tiles = round32(total_k) / kTile;
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
