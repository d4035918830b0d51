// Varlen (packed-segment) attention for edge-set attention on gfx950: the
// C ABI entry points, the edge-mask (share-an-endpoint) bf16 kernels, the
// fp32 kernels (dense and edge mask) and the per-call prep.  Dense bf16
// attention dispatches to esa_attn_dense.hip, the node-mode CSR mask to
// esa_graph_attn.hip.
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
// Edge-mask tiling.  Tokens are cut into 32-token tiles aligned to the
// global token index; a tile may straddle segments, which the per-element
// validity test (partner token in the lane's segment) resolves.  A wave owns
// one outer tile and two heads; the four waves of a 256-thread block are the
// four tiles of a 128-token group and walk on their own: each visits only
// the partner tiles whose node sets may meet its tile (node-range and 64-bit
// signature test of per-tile metadata), staging them into its own
// double-buffered LDS region.  The mask of a visited tile is evaluated once
// per wave into an additive bias (0 or -inf per score) that seeds the score
// MFMA of each head.  Groups are dispatched longest-first (a per-call plan
// kernel sorts them by the number of partner tiles).
//
// Register layout (head_dim = 16 = the MFMA K of 32x32x16):
//   S^T = K_tile * Q_tile^T : lane l owns query column l%32; its 16 fp32
//   accumulators hold keys k0 + 16(r>>3) + 8(l>>5) + (r&7).  Rows of the K
//   operand are permuted (bits 2 and 3 of the row swapped) to make that
//   mapping, so each half-wave's 8 P values are 8 consecutive keys — exactly
//   the B operand of the P V product, with no data movement.
//   O^T = [V^T ; 1] * P^T : rows 0..15 are the output dims, rows 16..31 are
//   ones, so the MFMA also produces the softmax row sum.  Softmax statistics
//   stay per lane (one query per lane).  Operands with the token dimension
//   in the MFMA K slots (V^T, K^T, Q^T, dO^T) come from LDS transpose reads
//   of rows staged split by dims half.
//   The dK/dV pass keeps keys on lanes; per-query row statistics (LSE, D)
//   enter through an extra MFMA whose A operand carries (hi, lo) bf16 halves
//   of -LSE/c and -D per row and whose B operand is a column of ones: it
//   broadcasts each row's value across the lanes in fp32 at no VALU cost.
//
// Softmax reference point.  By Cauchy-Schwarz every score of query i obeys
// c*|S_ij| <= c*|q_i|*max_j|k_j| =: b_i (c = scale*log2 e).  When b_i <= 60 for
// every query of a wave, exp2(c*S_ij - b_i) lies in [2^-120, 1]: no overflow,
// no underflow, so softmax(S) = p / sum(p) with the fixed reference b_i is
// exact up to rounding and needs no running max and no rescaling.  Waves with
// a larger bound take the online (running-max) path.
//
// Global loads go through buffer resources with the tensor's byte size as
// range: the hardware returns 0 for any part of a load past the end, so tiles
// that run past the last token need no index clamping.
#include <mutex>
#include <type_traits>

#include "esa_attn_tiles.h"
#include "esa_attn_dense.h"
#include "esa_common.h"
#include "esa_graph_attn.h"
#include "esa_profile.h"
#include "../../include/esa_hip.h"

namespace {


// The outer tile a wave owns: per-lane partner range and wave-level bounds.
struct OuterTile {
  bool active;         // tile starts before `total`
  int oi;              // this lane's outer token
  bool valid;          // oi < total
  int oc;              // oi clamped into [0, total)
  int plo, phi;        // partner range of the lane's segment (empty when !valid)
  int plo_max, phi_min;
  int pt_beg, pt_end;  // partner tiles this wave visits
};

DEVI int wave_reduce_max(int x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = max(x, __shfl_xor(x, o));
  return x;
}
DEVI int wave_reduce_min(int x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = min(x, __shfl_xor(x, o));
  return x;
}

// bounds[t] = partner range [cu_inner[s], cu_inner[s+1]) of token t's segment
// s (precomputed once per call, so no kernel searches cu_seqlens).  Lanes
// 32..63 mirror lanes 0..31.
DEVI OuterTile outer_tile(const int2* __restrict__ bounds, int total, int o0, int col) {
  OuterTile t;
  t.oi = o0 + col;
  t.active = o0 < total;
  t.valid = t.oi < total;
  t.oc = t.valid ? t.oi : max(total - 1, 0);
  t.plo = t.phi = 0;
  t.plo_max = INT_MAX;
  t.phi_min = INT_MIN;
  t.pt_beg = t.pt_end = 0;
  if (!t.active) return t;
  const int2 b = bounds[t.oc];
  if (t.valid) { t.plo = b.x; t.phi = b.y; }
  t.plo_max = wave_reduce_max(t.valid ? b.x : INT_MIN);
  t.phi_min = wave_reduce_min(t.valid ? b.y : INT_MAX);
  const int lo = wave_reduce_min(t.valid ? b.x : INT_MAX);
  const int hi = wave_reduce_max(t.valid ? b.y : INT_MIN);
  t.pt_beg = lo >> 5;
  t.pt_end = max(t.pt_beg, (hi + kTile - 1) >> 5);
  return t;
}

// ---------------------------------------------------------------- tile walk
//
// Each wave walks, on its own, only the partner tiles whose node sets may
// meet its outer tile (node range and 64-bit signature test of the per-tile
// metadata; 64 candidates per ballot), staging them into its own
// double-buffered LDS region.  No block barrier: a wave never waits for
// another wave's tiles.

constexpr int kWaitVmem = 0x0F70;   // s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15) (gfx9 encoding)

// LDS writes of one wave become visible to its other lanes in issue order;
// the fences only keep the compiler from moving LDS accesses across.
DEVI void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Walk over n partner tiles: next(waves) returns the next tile index (in
// order; past the end it repeats the last one) and its wave mask,
// gload(pt) fetches a tile's staging registers, lstore(buf, regs) writes
// them to LDS buffer `buf`, body(pt, buf, waves) consumes a staged tile,
// sync() orders LDS writes before reads.  Two LDS buffers and two tiles'
// loads in flight: tile i+2 is requested before tile i is consumed and tile
// i+1 is written to LDS after it.  Loads are issued unconditionally (past the
// end they re-read the last tile and are not consumed) so each wait covers
// exactly the older load; the loop is unrolled by two so the staging
// registers never move (a register copy would wait for its load) and the
// LDS buffer index is a constant in each half.
template <class Next, class Load, class Store, class Sync, class Body>
DEVI void tile_pipeline(int n, Next next, Load gload, Store lstore, Sync sync, Body body) {
  if (n <= 0) return;
  uint32_t w0 = 0, w1 = 0;
  int p0 = next(w0);
  const auto s0 = gload(p0);
  int p1 = next(w1);
  auto sb = gload(p1);
  decltype(sb) sa;
  lstore(0, s0);
  sync();
  for (int i = 0; i < n; i += 2) {
    // buffer 0 holds tile i (p0, w0); sb is tile i+1 (p1, w1), in flight
    uint32_t w2 = 0;
    const int p2 = next(w2);
    sa = gload(p2);
    body(p0, 0, w0);
    if (i + 1 < n) lstore(1, sb);
    sync();
    if (i + 1 >= n) break;
    // buffer 1 holds tile i+1 (p1, w1); sa is tile i+2 (p2, w2), in flight
    uint32_t w3 = 0;
    const int p3 = next(w3);
    sb = gload(p3);
    body(p1, 1, w1);
    if (i + 2 < n) lstore(0, sa);
    sync();
    p0 = p2; w0 = w2;
    p1 = p3; w1 = w3;
  }
}

// The walk starts with every earlier vector-memory load complete: a
// prologue load still pending inside the loop would be waited for with
// vmcnt(0), which also waits for the prefetches in flight.
template <class Load, class Store, class Body>
DEVI void wave_tile_walk(int pt_beg, int pt_end, int4 own, const int4* __restrict__ meta, int lane, Load gload,
                         Store lstore, Body body) {
  __builtin_amdgcn_s_waitcnt(kWaitVmem);
  for (int base = pt_beg; base < pt_end; base += 64) {
    const int x = base + lane;
    bool need = false;
    if (x < pt_end) need = tiles_may_touch(own, meta[x]);
    unsigned long long bits = __ballot(need);
    int last = base;
    tile_pipeline(__popcll(bits), [&](uint32_t& w) {
      w = 0xfu;
      if (bits) {
        last = base + __builtin_ctzll(bits);
        bits &= bits - 1;
      }
      return last;
    }, gload, lstore, wave_sync, body);
  }
}

struct AttnArgs {
  const bf16* q; const bf16* k; const bf16* v; const bf16* out; const bf16* dout;
  const float* lse;         // [H][total_q] natural log (forward output / backward input)
  const uint2* aux;         // dK/dV pass: per (head, query) packed bf16 (hi, lo) of -LSE2/c and of -D
  uint2* aux_out;           // key-list dQ pass: writes aux (it reads dO, O and LSE of its queries anyway)
  const float* knorm;       // forward: max |k| per (head, key tile) [H][tk_tiles]
  const int* cu_q; const int* cu_k; int nseg;
  int total_q, total_k, heads, tq_pad, tk_tiles;
  float c;                  // softmax_scale * log2(e)
  float scale;
  const int2* nodes; const int4* meta;   // masked mode: per-token node pairs (padded), per-tile metadata
  const int4* plan;         // per block group: (group, first partner tile, end partner tile, -)
  const int* count;         // walk kernels: number of plan entries (the overflow list)
  const int2* bounds;       // per outer token: partner range of its segment
  const int* info;          // key lists: per outer tile, the number of partners (-1: group overflowed)
  const int* ids;           // key lists: per outer tile, kListCap partner token ids (-1 pads)
  const uint32_t* bits;     // key lists: per outer tile, [kListCap / 32][32] mask words
  // Edge plans: the key tiles' own lists and overflow groups, used by the dK/dV
  // passes unless *sym (the plan's flag: query and key segments coincide, the
  // mask is symmetric and the query tiles' lists serve the key tiles).
  const int* sym;
  const int* kinfo; const int* kids; const uint32_t* kbits; const int4* kover; const int* kcount;
  bf16* o; float* lse_out;  // forward outputs
  bf16* dq; bf16* dk; bf16* dv;
};

// Staging source of one lane: a buffer resource plus this lane's 16-byte
// chunk of a tile.  Loads past the resource return zeros without touching
// memory (also the empty resource of a wave without a role).
struct StageSrc {
  rsrc_t rsrc;
  uint32_t base, step;   // byte offset of this lane's chunk in tile 0; bytes per tile
  DEVI uint32_t offset(int pt) const { return base + (uint32_t)pt * step; }
  DEVI i32x4 load(int pt) const { return bload(rsrc, offset(pt)); }
};

// Token rows [T][H][16] bf16: lane l reads half (l & 1) of token l >> 1.
// Per-token 8-byte records [T]: lanes 0..15 read two records each; the other
// lanes read beyond the resource (zeros).
DEVI StageSrc rows_src(const void* p, int bytes, int H, int head, int lane) {
  return StageSrc{make_rsrc(p, (uint32_t)bytes),
                  ((uint32_t)(lane >> 1) * H + head) * (kHd * 2) + 16u * (lane & 1), (uint32_t)(kTile * H * kHd * 2)};
}
DEVI StageSrc records_src(const void* p, int n_records, int lane) {
  return StageSrc{make_rsrc(p, (uint32_t)n_records * 8u), lane < 16 ? 16u * lane : 0x80000000u, (uint32_t)kTile * 8u};
}

// LDS writes of a staged 32-token tile: rows [token][16] (padded stride) and
// 8-byte records (lanes 0..15).
DEVI void put_rows(bf16* rows, i32x4 v, int lane) {
  *reinterpret_cast<i32x4*>(&rows[(lane >> 1) * kRowStride + 8 * (lane & 1)]) = v;
}
template <class R>
DEVI void put_records(R* rec, i32x4 v, int lane) {
  if (lane < 16) *reinterpret_cast<i32x4*>(&rec[2 * lane]) = v;
}


// ======================================================================== edge-mask forward, heads in pairs
// One wave = one 32-query tile and kEdgeHeads heads of it (the four waves of
// a block are four tiles of a 128-token group and walk on their own, as in
// the masked walk above).  The mask of a candidate key tile is evaluated
// once, into an additive bias of 0 or -inf per score, which is the
// accumulator seed of every head's score MFMAs: masking is free per head,
// and the wave's fixed costs (segment bounds, tile metadata, the candidate
// ballot) are shared by its heads.  Each candidate tile stages K rows and V
// rows (split by dims half; the [V^T ; 1] operands come from LDS transpose
// reads) of all heads of the wave plus the 32 node pairs.

#ifndef ESA_EDGE_HEADS
#define ESA_EDGE_HEADS 2
#endif
constexpr int kEdgeHeads = ESA_EDGE_HEADS;
constexpr int kTileHalf = kTile * 8;   // bf16 per dims half of a split-row tile

// Bias (0 keep / -inf drop) of this lane's 16 accumulator rows (partner
// token p0 + row_local(r, half)) against the lane's own token: keep if the
// partner shares an endpoint with it, lies in its segment and is not the
// token itself.  Segment bounds and the diagonal are only tested on tiles
// that straddle a segment bound of the wave or hold its own tokens.
DEVI f32x16 edge_bias(const OuterTile& ot, int p0, int o0, int half, const int2* sn, int2 own) {
  int2 pn[16];
  lds_nodes16(sn, half, pn);
  f32x16 b;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const uint32_t d = min(min((uint32_t)(pn[r].x ^ own.x), (uint32_t)(pn[r].x ^ own.y)),
                           min((uint32_t)(pn[r].y ^ own.x), (uint32_t)(pn[r].y ^ own.y)));
    b[r] = d == 0u ? 0.f : -INFINITY;
  }
  if (!(p0 >= ot.plo_max && p0 + kTile <= ot.phi_min) || p0 == o0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int p = p0 + row_local(r, half);
      b[r] = (p >= ot.plo && p < ot.phi && p != ot.oi) ? b[r] : -INFINITY;
    }
  }
  return b;
}

// Token rows [T][H][16] bf16 for split-row staging: lane l reads dims half
// l >> 5 of token l & 31 (lanes 0..31 write 512 contiguous LDS bytes).
DEVI StageSrc split_rows_src(const void* p, int bytes, int H, int head, int lane) {
  return StageSrc{make_rsrc(p, (uint32_t)bytes),
                  ((uint32_t)(lane & 31) * H + head) * (kHd * 2) + 16u * (lane >> 5), (uint32_t)(kTile * H * kHd * 2)};
}

template <int NH>
struct StageEdge { i32x4 k[NH], v[NH], n; };

#ifndef ESA_EDGE_WAVES
#define ESA_EDGE_WAVES 2
#endif
DEVI void edge_fwd_group(const AttnArgs& a, int item, int hg, const bf16* sOnes) {
  constexpr int NH = kEdgeHeads;
  __shared__ __align__(16) bf16 sK[kWaves][2][NH][kTile * kRowStride];   // K rows [key][16]
  __shared__ __align__(16) bf16 sV[kWaves][2][NH][2 * kTileHalf];        // V rows split by dims half
  __shared__ __align__(16) int2 sN[kWaves][2][kTile];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5, c16 = lane & 15, grp = lane >> 4;
  const int H = a.heads;
  const int h0 = hg * NH;
  const int nh = min(NH, H - h0);   // heads of this wave
  const int4 pl = a.plan[item];
  const int t0 = pl.x * kGroupTok, o0 = t0 + wave * kTile;

  const OuterTile ot = outer_tile(a.bounds, a.total_q, o0, col);
  const int2 qn = a.nodes[ot.oc];
  const int4 own = ot.active ? a.meta[o0 / kTile] : no_touch();
  bf16x8 qh[NH], ql[NH];
  float bmax = a.knorm ? 0.f : INFINITY;   // without key norms: the online path
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    const int hc = min(h0 + u, H - 1);
    const bf16x8 qf = *reinterpret_cast<const bf16x8*>(a.q + ((size_t)ot.oc * H + hc) * kHd + 8 * half);
    if (ot.active && a.knorm) {
      // bound c |q| max|k| over the keys this wave visits
      float qq = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) qq = fmaf((float)qf[e], (float)qf[e], qq);
      qq += __shfl_xor(qq, 32);
      float km = 0.f;
      for (int t = ot.pt_beg + lane; t < ot.pt_end; t += 64) km = fmaxf(km, a.knorm[(size_t)hc * a.tk_tiles + t]);
      km = wave_max(km);
      bmax = fmaxf(bmax, ot.valid ? a.c * sqrtf(qq) * km : 0.f);
    }
    split_scaled(qf, a.c, qh[u], ql[u]);
  }
  const bool fixed_ref = __builtin_amdgcn_readfirstlane((int)(wave_max(bmax) <= kStaticBound)) != 0;

  float m_run[NH];
  f32x16 acc[NH];
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    m_run[u] = fixed_ref ? 0.f : -INFINITY;
    acc[u] = f32x16{};
  }
  const int kv_bytes = a.total_k * H * kHd * 2;
  StageSrc sk[NH], sv[NH];
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    const int hc = min(h0 + u, H - 1);
    sk[u] = rows_src(a.k, kv_bytes, H, hc, lane);
    sv[u] = split_rows_src(a.v, kv_bytes, H, hc, lane);
  }
  const StageSrc sn = records_src(a.nodes, a.tq_pad, lane);
  auto run = [&](auto online_tag) {
    constexpr bool ONLINE = decltype(online_tag)::value;
    auto body = [&](int pt, int cur, uint32_t) {
      if (!(pt >= ot.pt_beg && pt < ot.pt_end)) return;
      const int k0 = pt * kTile;
      const f32x16 bias = edge_bias(ot, k0, o0, half, sN[wave][cur], qn);
#pragma unroll
      for (int u = 0; u < NH; ++u) {
        if (u >= nh) break;   // wave-uniform
        const bf16x8 kr = lds8(&sK[wave][cur][u][kperm(col) * kRowStride + 8 * half]);
        f32x16 s = mfma32(kr, ql[u], mfma32(kr, qh[u], bias));
        if (ONLINE) {
          float mt = s[0];
#pragma unroll
          for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
          mt = fmaxf(mt, __shfl_xor(mt, 32));
          const float m_new = fmaxf(m_run[u], mt);
          if (__ballot(m_new > m_run[u])) {
            const float alpha = fast_exp2(m_run[u] - (m_new == -INFINITY ? 0.f : m_new));
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[u][r] *= alpha;
            m_run[u] = m_new;
          }
        }
        float p[16];
        const float m_use = ONLINE ? (m_run[u] == -INFINITY ? 0.f : m_run[u]) : 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = fast_exp2(ONLINE ? s[r] - m_use : s[r]);
        bf16x8 vt0, vt1;
        tr_rows32<kTileHalf>(sV[wave][cur][u], 0, sOnes, c16, grp, vt0, vt1);
        acc[u] = mfma32(vt0, cvt8(p), acc[u]);
        acc[u] = mfma32(vt1, cvt8(p + 8), acc[u]);
      }
    };
    wave_tile_walk(ot.pt_beg, ot.pt_end, own, a.meta, lane,
                   [&](int pt) {
                     StageEdge<NH> g;
#pragma unroll
                     for (int u = 0; u < NH; ++u) {
                       g.k[u] = sk[u].load(pt);
                       g.v[u] = sv[u].load(pt);
                     }
                     g.n = sn.load(pt);
                     return g;
                   },
                   [&](int st, const StageEdge<NH>& g) {
#pragma unroll
                     for (int u = 0; u < NH; ++u) {
                       put_rows(sK[wave][st][u], g.k[u], lane);
                       put_half<kTileHalf>(sV[wave][st][u], lane & 31, lane >> 5, g.v[u]);
                     }
                     put_records(sN[wave][st], g.n, lane);
                   },
                   body);
  };
  if (fixed_ref)
    run(std::integral_constant<bool, false>{});
  else
    run(std::integral_constant<bool, true>{});
  if (!ot.valid) return;
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    if (u >= nh) break;
    const int h = h0 + u;
    const float l = acc[u][8];   // a ones row of [V^T; 1] P^T: the softmax row sum
    store_rows8(a.o + ((size_t)ot.oi * H + h) * kHd, acc[u], l > 0.f ? 1.f / l : 0.f, half);
    if (half == 0)
      a.lse_out[(size_t)h * a.total_q + ot.oi] = l > 0.f ? (m_run[u] + fast_log2(l)) * kLn2 : -INFINITY;
  }
}

// The walk kernels run over a list of groups with a device-side count (the
// groups whose key lists overflow): a block loops over list items, so a small
// fixed grid serves any count and costs little when the list is empty.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(ESA_EDGE_WAVES))) void edge_fwd_kernel(
    const AttnArgs a) {
  __shared__ __align__(16) bf16 sOnes[4];   // the ones rows of [V^T ; 1]
  const int n_hg = (a.heads + kEdgeHeads - 1) / kEdgeHeads, hg = blockIdx.x % n_hg;
  const int n_items = *a.count;
  if ((int)blockIdx.x / n_hg >= n_items) return;
  if (threadIdx.x < 4) sOnes[threadIdx.x] = (bf16)1.f;
  __syncthreads();
  for (int item = blockIdx.x / n_hg; item < n_items; item += gridDim.x / n_hg) edge_fwd_group(a, item, hg, sOnes);
}

// ======================================================================== edge-mask dQ pass
// One wave = one 32-query tile and kEdgeHeads heads of it, as the forward:
// dQ = scale * dS K with dS = P * (dP - D), P recomputed from the saved
// LSE.  The mask bias of a candidate key tile is evaluated once and seeds
// every head's score MFMA; K and V are staged as split rows, K^T comes from
// LDS transpose reads.

#ifndef ESA_EDGE_WAVES_DQ
#define ESA_EDGE_WAVES_DQ 2
#endif
DEVI void edge_dq_group(const AttnArgs& a, int item, int hg) {
  constexpr int NH = kEdgeHeads;
  __shared__ __align__(16) bf16 sK[kWaves][2][NH][2 * kTileHalf];   // K rows split by dims half
  __shared__ __align__(16) bf16 sV[kWaves][2][NH][2 * kTileHalf];   // V rows split by dims half
  __shared__ __align__(16) int2 sN[kWaves][2][kTile];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5, c16 = lane & 15, grp = lane >> 4;
  const int H = a.heads;
  const int h0 = hg * NH;
  const int nh = min(NH, H - h0);   // heads of this wave
  const int4 pl = a.plan[item];
  const int o0 = pl.x * kGroupTok + wave * kTile;

  const OuterTile ot = outer_tile(a.bounds, a.total_q, o0, col);
  const int2 qn = a.nodes[ot.oc];
  const int4 own = ot.active ? a.meta[o0 / kTile] : no_touch();
  bf16x8 qf[NH], dof[NH];
  float dsum[NH], lse2q[NH];
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    const int hc = min(h0 + u, H - 1);
    const size_t row = ((size_t)ot.oc * H + hc) * kHd + 8 * half;
    qf[u] = *reinterpret_cast<const bf16x8*>(a.q + row);
    dof[u] = *reinterpret_cast<const bf16x8*>(a.dout + row);
    const bf16x8 of = *reinterpret_cast<const bf16x8*>(a.out + row);
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) d = fmaf((float)dof[u][e], (float)of[e], d);
    dsum[u] = d + __shfl_xor(d, 32);
    const float lq = a.lse[(size_t)hc * a.total_q + ot.oc];
    lse2q[u] = lq == -INFINITY ? INFINITY : lq * kLog2e;
  }

  f32x16 acc[NH];
#pragma unroll
  for (int u = 0; u < NH; ++u) acc[u] = f32x16{};
  const f32x16 zero = {};
  auto body = [&](int pt, int cur, uint32_t) {
    if (!(pt >= ot.pt_beg && pt < ot.pt_end)) return;
    const int k0 = pt * kTile;
    const f32x16 bias = edge_bias(ot, k0, o0, half, sN[wave][cur], qn);
#pragma unroll
    for (int u = 0; u < NH; ++u) {
      if (u >= nh) break;   // wave-uniform
      const f32x16 s = mfma32(half_row8<kTileHalf>(sK[wave][cur][u], kperm(col), half), qf[u], bias);
      const f32x16 dp = mfma32(half_row8<kTileHalf>(sV[wave][cur][u], kperm(col), half), dof[u], zero);
      float ds[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) ds[r] = fast_exp2(fmaf(s[r], a.c, -lse2q[u])) * (dp[r] - dsum[u]);
      bf16x8 kt0, kt1;
      tr_rows32<kTileHalf>(sK[wave][cur][u], 0, nullptr, c16, grp, kt0, kt1);
      acc[u] = mfma32(kt0, cvt8(ds), acc[u]);
      acc[u] = mfma32(kt1, cvt8(ds + 8), acc[u]);
    }
  };
  const int kv_bytes = a.total_k * H * kHd * 2;
  StageSrc sk[NH], sv[NH];
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    const int hc = min(h0 + u, H - 1);
    sk[u] = split_rows_src(a.k, kv_bytes, H, hc, lane);
    sv[u] = split_rows_src(a.v, kv_bytes, H, hc, lane);
  }
  const StageSrc sn = records_src(a.nodes, a.tq_pad, lane);
  wave_tile_walk(ot.pt_beg, ot.pt_end, own, a.meta, lane,
                 [&](int pt) {
                   StageEdge<NH> g;
#pragma unroll
                   for (int u = 0; u < NH; ++u) {
                     g.k[u] = sk[u].load(pt);
                     g.v[u] = sv[u].load(pt);
                   }
                   g.n = sn.load(pt);
                   return g;
                 },
                 [&](int st, const StageEdge<NH>& g) {
#pragma unroll
                   for (int u = 0; u < NH; ++u) {
                     put_half<kTileHalf>(sK[wave][st][u], lane & 31, lane >> 5, g.k[u]);
                     put_half<kTileHalf>(sV[wave][st][u], lane & 31, lane >> 5, g.v[u]);
                   }
                   put_records(sN[wave][st], g.n, lane);
                 },
                 body);
  if (!ot.valid) return;
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    if (u >= nh) break;
    store_rows8(a.dq + ((size_t)ot.oi * H + h0 + u) * kHd, acc[u], a.scale, half);
  }
}

// ======================================================================== edge-mask dK/dV pass
// One wave = one 32-key tile (keys on lanes, queries in rows) and
// kEdgeHeadsKv heads of it: dV = P^T dO, dK = scale * dS^T Q.  Row
// statistics (-LSE2/c, -D as bf16 hi/lo pairs) enter through MFMAs against a
// ones column; the mask bias of a candidate query tile, evaluated once per
// tile, seeds every head's -LSE2/c one.  Q and dO are staged as split rows,
// Q^T and dO^T come from LDS transpose reads.

#ifndef ESA_EDGE_HEADS_KV
#define ESA_EDGE_HEADS_KV 1
#endif
constexpr int kEdgeHeadsKv = ESA_EDGE_HEADS_KV;
#ifndef ESA_EDGE_WAVES_DKDV
#define ESA_EDGE_WAVES_DKDV 2
#endif

template <int NH>
struct StageKv { i32x4 q[NH], d[NH], x[NH], n; };

DEVI void edge_dkdv_group(const AttnArgs& a, int item, int hg) {
  constexpr int NH = kEdgeHeadsKv;
  __shared__ __align__(16) bf16 sQ[kWaves][2][NH][2 * kTileHalf];    // Q rows split by dims half
  __shared__ __align__(16) bf16 sDO[kWaves][2][NH][2 * kTileHalf];   // dO rows split by dims half
  __shared__ __align__(16) uint2 sAux[kWaves][2][NH][kTile];         // row-statistic MFMA operands
  __shared__ __align__(16) int2 sN[kWaves][2][kTile];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5, c16 = lane & 15, grp = lane >> 4;
  const int H = a.heads;
  const int h0 = hg * NH;
  const int nh = min(NH, H - h0);   // heads of this wave
  const int4 pl = a.plan[item];
  const int o0 = pl.x * kGroupTok + wave * kTile;

  const OuterTile ot = outer_tile(a.bounds, a.total_k, o0, col);
  bf16x8 kf[NH], vf[NH];
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    const size_t row = ((size_t)ot.oc * H + min(h0 + u, H - 1)) * kHd + 8 * half;
    kf[u] = *reinterpret_cast<const bf16x8*>(a.k + row);
    vf[u] = *reinterpret_cast<const bf16x8*>(a.v + row);
  }
  // B operand of the row-statistic MFMAs: ones in slots 0 and 1 (half 0).
  bf16x8 ones2 = {};
  if (half == 0) { ones2[0] = (bf16)1.f; ones2[1] = (bf16)1.f; }
  const int2 kn = a.nodes[ot.oc];
  const int4 own = ot.active ? a.meta[o0 / kTile] : no_touch();

  f32x16 dva[NH], dka[NH];
#pragma unroll
  for (int u = 0; u < NH; ++u) dva[u] = dka[u] = f32x16{};
  const f32x16 zero = {};
  auto body = [&](int pt, int cur, uint32_t) {
    if (!(pt >= ot.pt_beg && pt < ot.pt_end)) return;
    const int q0 = pt * kTile;
    const f32x16 bias = edge_bias(ot, q0, o0, half, sN[wave][cur], kn);
#pragma unroll
    for (int u = 0; u < NH; ++u) {
      if (u >= nh) break;   // wave-uniform
      const uint2 ax = sAux[wave][cur][u][kperm(col)];
      const bf16x8 aux_s = as_bf16x8(i32x4{(int)ax.x, 0, 0, 0});
      const bf16x8 aux_d = as_bf16x8(i32x4{(int)ax.y, 0, 0, 0});
      // S' = Q K^T - LSE2/c + bias and dP' = dO V^T - D, rows = queries, lanes = keys.
      const f32x16 s =
          mfma32(half_row8<kTileHalf>(sQ[wave][cur][u], kperm(col), half), kf[u], mfma32(aux_s, ones2, bias));
      const f32x16 dp =
          mfma32(half_row8<kTileHalf>(sDO[wave][cur][u], kperm(col), half), vf[u], mfma32(aux_d, ones2, zero));
      float p[16], ds[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = fast_exp2(s[r] * a.c);
        ds[r] = p[r] * dp[r];
      }
      bf16x8 d0, d1, q0t, q1t;
      tr_rows32<kTileHalf>(sDO[wave][cur][u], 0, nullptr, c16, grp, d0, d1);
      tr_rows32<kTileHalf>(sQ[wave][cur][u], 0, nullptr, c16, grp, q0t, q1t);
      dva[u] = mfma32(d0, cvt8(p), dva[u]);
      dva[u] = mfma32(d1, cvt8(p + 8), dva[u]);
      dka[u] = mfma32(q0t, cvt8(ds), dka[u]);
      dka[u] = mfma32(q1t, cvt8(ds + 8), dka[u]);
    }
  };
  const int q_bytes = a.total_q * H * kHd * 2;
  StageSrc sq[NH], sd[NH], sa[NH];
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    const int hc = min(h0 + u, H - 1);
    sq[u] = split_rows_src(a.q, q_bytes, H, hc, lane);
    sd[u] = split_rows_src(a.dout, q_bytes, H, hc, lane);
    sa[u] = records_src(a.aux + (size_t)hc * a.tq_pad, a.tq_pad, lane);
  }
  const StageSrc sn = records_src(a.nodes, a.tq_pad, lane);
  wave_tile_walk(ot.pt_beg, ot.pt_end, own, a.meta, lane,
                 [&](int pt) {
                   StageKv<NH> g;
#pragma unroll
                   for (int u = 0; u < NH; ++u) {
                     g.q[u] = sq[u].load(pt);
                     g.d[u] = sd[u].load(pt);
                     g.x[u] = sa[u].load(pt);
                   }
                   g.n = sn.load(pt);
                   return g;
                 },
                 [&](int st, const StageKv<NH>& g) {
#pragma unroll
                   for (int u = 0; u < NH; ++u) {
                     put_half<kTileHalf>(sQ[wave][st][u], lane & 31, lane >> 5, g.q[u]);
                     put_half<kTileHalf>(sDO[wave][st][u], lane & 31, lane >> 5, g.d[u]);
                     put_records(sAux[wave][st][u], g.x[u], lane);
                   }
                   put_records(sN[wave][st], g.n, lane);
                 },
                 body);
  if (!ot.valid) return;
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    if (u >= nh) break;
    const int h = h0 + u;
    store_rows8(a.dv + ((size_t)ot.oi * H + h) * kHd, dva[u], 1.f, half);
    store_rows8(a.dk + ((size_t)ot.oi * H + h) * kHd, dka[u], a.scale, half);
  }
}

// The backward walks over the overflowing groups in one launch: both read only the row statistics the list
// dQ pass wrote, and they write disjoint outputs (dQ of the query tiles' groups, dK / dV of the key tiles'),
// so blocks [0, dq_blocks) take the dQ walk and the rest the dK/dV walk.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(
    ESA_EDGE_WAVES_DQ < ESA_EDGE_WAVES_DKDV ? ESA_EDGE_WAVES_DQ : ESA_EDGE_WAVES_DKDV))) void edge_bwd_walk_kernel(
    const AttnArgs adq, const AttnArgs akv, int dq_blocks) {
  if ((int)blockIdx.x < dq_blocks) {
    const int n_hg = (adq.heads + kEdgeHeads - 1) / kEdgeHeads, hg = blockIdx.x % n_hg;
    const int n_items = *adq.count;
    for (int item = blockIdx.x / n_hg; item < n_items; item += dq_blocks / n_hg) edge_dq_group(adq, item, hg);
    return;
  }
  AttnArgs a = akv;
  if (akv.sym && !*akv.sym) {   // the key tiles' own overflow groups
    a.plan = akv.kover;
    a.count = akv.kcount;
  }
  const int b = blockIdx.x - dq_blocks, nb = gridDim.x - dq_blocks;
  const int n_hg = (a.heads + kEdgeHeadsKv - 1) / kEdgeHeadsKv, hg = b % n_hg;
  const int n_items = *a.count;
  for (int item = b / n_hg; item < n_items; item += nb / n_hg) edge_dkdv_group(a, item, hg);
}

// ======================================================================== edge-mask key lists
// The walk kernels above evaluate the mask of every candidate partner tile
// once per head group.  The key lists evaluate it once per call: per 32-token
// outer tile, the union of the partner tokens that any of its tokens attends
// (shares an endpoint, lies in its segment, is not itself), in ascending token
// order, and per outer token one mask bit per union entry.  The list kernels
// below visit ceil(union / 32) compact tiles per outer tile, gather the
// partner rows by id and build a tile's bias from one 32-bit word per lane.
// When the query and key segments coincide the mask is symmetric and the
// dK/dV pass reads the query tiles' lists.
//
// Capacity: kListCap partners per outer tile.  A 128-token group with a tile
// past capacity gets info -1 on its four tiles and goes to an overflow list,
// which the walk kernels process.

#ifndef ESA_LIST_CAP
#define ESA_LIST_CAP 384
#endif
constexpr int kListCap = ESA_LIST_CAP;
static_assert(kListCap % kTile == 0, "list capacity in whole tiles");

struct ListArgs {
  const int2* nodes; const int4* meta;
  int total, n_groups;          // outer (= partner) tokens and 128-token groups per direction
  const int2* bounds[2];        // per outer token: partner range of its segment (0: queries, 1: keys)
  int* info[2]; int* ids[2]; uint32_t* bits[2];
  int4* over[2]; int* over_count[2];
};

// 32 x 32 bit-matrix transpose across lanes 0..31 (and, separately, 32..63):
// lane r holds row r (bit c = element (r, c)) and receives column r.  Five
// butterfly stages swap the off-diagonal blocks of size 16, 8, 4, 2, 1.
DEVI uint32_t transpose32(uint32_t x, int lane) {
  uint32_t m = 0x0000FFFFu;
#pragma unroll
  for (int j = 16; j > 0; j >>= 1, m ^= m << j) {
    const uint32_t t = (uint32_t)__shfl_xor((int)x, j);
    x = (lane & j) ? ((x & ~m) | ((t >> j) & m)) : ((x & m) | ((t & m) << j));
  }
  return x;
}

constexpr int kHashSlots = 128;   // per wave: the outer tile's <= 64 node ids, load <= 1/2
DEVI int node_slot(int node) { return (int)(((uint32_t)node * 2654435761u) >> 25); }

// Mask of the outer tile's tokens that have `node` as an endpoint (0 if none).
DEVI uint32_t node_lookup(const int* keys, const uint32_t* masks, int node) {
  if (node < 0) return 0u;
  int h = node_slot(node);
  for (int i = 0; i < kHashSlots; ++i) {
    const int k = keys[h];
    if (k == node) return masks[h];
    if (k < 0) return 0u;
    h = (h + 1) & (kHashSlots - 1);
  }
  return 0u;
}

// One block = one 128-token group of one direction, one wave per outer tile.
// A wave hashes its tile's node ids (node -> mask of the tile's tokens with
// that endpoint, open addressing in LDS) and records the runs of its tokens
// that share a partner range (one per segment).  Then, per batch of 64
// partner tiles, the candidates (node-range and signature test of the tile
// metadata, as the walk kernels) are processed in three data-parallel steps:
//  A. every candidate token's mask over the outer tokens: the OR of its two
//     endpoints' lookups, cut to the runs whose range holds it and off the
//     diagonal (two candidates per step, 16 candidates' loads in flight);
//  B. a wave prefix scan of the candidates' union sizes gives every kept
//     token its list position: ids to global, masks to LDS;
// and at the end, C. each run of 32 entries is transposed into one word per
// outer token (bit k of word c: entry 32 c + k).
__global__ __launch_bounds__(256) void edge_lists_kernel(const ListArgs a) {
  constexpr int kBatch = 64;   // partner tiles per candidate ballot
  __shared__ int sKey[kWaves][kHashSlots];
  __shared__ uint32_t sQm[kWaves][kHashSlots];
  __shared__ int4 sRun[kWaves][kTile];               // (partner begin, partner end, token mask, -)
  __shared__ int sCand[kWaves][kBatch];              // candidate partner tiles of the batch
  __shared__ uint32_t sU[kWaves][kBatch];            // their unions (bit j: partner token j kept)
  __shared__ int sPre[kWaves][kBatch];               // their first list positions
  __shared__ uint32_t sKmA[kWaves][kBatch * kTile];  // masks of the batch's candidate tokens
  __shared__ uint32_t sKm[kWaves][kListCap];         // masks of the list entries
  __shared__ int s_over;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int dir = (int)blockIdx.x >= a.n_groups ? 1 : 0;
  const int g = (int)blockIdx.x - dir * a.n_groups;
  if (tid == 0) s_over = 0;
  __syncthreads();
  const int tile = g * kWaves + wave, o0 = tile * kTile;
  const OuterTile ot = outer_tile(a.bounds[dir], a.total, o0, col);
  int count = 0;
  bool over = false;
  if (ot.active) {
    const int2 qn = a.nodes[ot.oc];
    const int4 own = a.meta[tile];
    int* keys = sKey[wave];
    uint32_t* qm = sQm[wave];
    for (int i = lane; i < kHashSlots; i += 64) {
      keys[i] = -1;
      qm[i] = 0u;
    }
    wave_sync();
    const int node = half ? qn.y : qn.x;
    if (ot.valid && node >= 0) {
      int h = node_slot(node);
      for (int i = 0; i < kHashSlots; ++i) {
        const int prev = atomicCAS(&keys[h], -1, node);
        if (prev < 0 || prev == node) {
          atomicOr(&qm[h], 1u << col);
          break;
        }
        h = (h + 1) & (kHashSlots - 1);
      }
    }
    // runs of outer tokens with one partner range
    const int plo_prev = __shfl(ot.plo, max(col - 1, 0)), phi_prev = __shfl(ot.phi, max(col - 1, 0));
    const uint32_t vmask = (uint32_t)__ballot(ot.valid);
    const uint32_t starts = (uint32_t)__ballot(ot.valid && (col == 0 || ot.plo != plo_prev || ot.phi != phi_prev));
    const int nruns = __popc(starts);
    if (half == 0 && ((starts >> col) & 1u)) {
      const uint32_t later = starts & ~((2u << col) - 1u);   // starts after this lane (col = 31: none)
      const uint32_t below_end = later ? (1u << __builtin_ctz(later)) - 1u : 0xFFFFFFFFu;
      sRun[wave][__popc(starts & ((1u << col) - 1u))] =
          make_int4(ot.plo, ot.phi, (int)(below_end & ~((1u << col) - 1u) & vmask), 0);
    }
    wave_sync();

    // Mask over the outer tokens of partner token p with nodes pn.
    auto partner_mask = [&](int p, int2 pn) {
      uint32_t km = node_lookup(keys, qm, pn.x) | node_lookup(keys, qm, pn.y);
      if (km) {
        uint32_t sm = 0u;
        for (int k = 0; k < nruns; ++k) {
          const int4 r = sRun[wave][k];
          if (p >= r.x && p < r.y) sm |= (uint32_t)r.z;
        }
        km &= sm;
        if (p >= o0 && p < o0 + kTile) km &= ~(1u << (p - o0));
      }
      return km;
    };
    int* out_ids = a.ids[dir] + (size_t)tile * kListCap;
    uint32_t* out_bits = a.bits[dir] + (size_t)tile * kListCap;
    constexpr int kSteps = 8;   // steps (two candidates each) whose node loads are in flight together
    for (int base = ot.pt_beg; base < ot.pt_end; base += kBatch) {
      const int x = base + lane;
      const bool need = x < ot.pt_end && tiles_may_touch(own, a.meta[x]);
      const unsigned long long cand = __ballot(need);
      const int n = __popcll(cand);
      if (n == 0) continue;
      if (need) sCand[wave][__popcll(cand & ((1ull << lane) - 1ull))] = x;
      wave_sync();
      // A: candidate i = 2 r + half, its token col
      for (int r0 = 0; 2 * r0 < n; r0 += kSteps) {
        int2 pn[kSteps];
        int pt[kSteps];
#pragma unroll
        for (int k = 0; k < kSteps; ++k) {
          const int i = 2 * (r0 + k) + half;
          pt[k] = i < n ? sCand[wave][i] : -1;
          pn[k] = pt[k] >= 0 ? a.nodes[pt[k] * kTile + col] : make_int2(-1, -1);
        }
#pragma unroll
        for (int k = 0; k < kSteps; ++k) {
          if (2 * (r0 + k) >= n) break;   // wave-uniform
          const int i = 2 * (r0 + k) + half;
          const uint32_t km = pt[k] >= 0 ? partner_mask(pt[k] * kTile + col, pn[k]) : 0u;
          if (i < n) sKmA[wave][i * kTile + col] = km;
          const unsigned long long ub = __ballot(km != 0u);
          if (col == 0 && i < n) sU[wave][i] = (uint32_t)(ub >> (32 * half));
        }
      }
      wave_sync();
      // B: list positions
      const uint32_t ui = lane < n ? sU[wave][lane] : 0u;
      const int sz = __popc(ui);
      int incl = sz;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o);
        if (lane >= o) incl += t;
      }
      const int batch_total = __shfl(incl, 63);
      if (count + batch_total > kListCap) {
        over = true;
        break;
      }
      if (lane < n) sPre[wave][lane] = count + incl - sz;
      wave_sync();
      for (int r = 0; 2 * r < n; ++r) {
        const int i = 2 * r + half;
        if (i < n) {
          const uint32_t km = sKmA[wave][i * kTile + col];
          if (km) {
            const int e = sPre[wave][i] + __popc(sU[wave][i] & ((1u << col) - 1u));
            out_ids[e] = sCand[wave][i] * kTile + col;
            sKm[wave][e] = km;
          }
        }
      }
      count += batch_total;
      wave_sync();
    }
    if (!over) {
      // C: one word per outer token per 32 entries
      for (int c = 0; c * kTile < count; ++c) {
        const int e = c * kTile + col;
        const uint32_t w = transpose32(e < count ? sKm[wave][e] : 0u, lane);
        if (half == 0) out_bits[c * kTile + col] = w;
      }
      const int padded = (count + kTile - 1) & ~(kTile - 1);
      if (lane < padded - count) out_ids[count + lane] = -1;
    }
  }
  if (over && lane == 0) s_over = 1;
  __syncthreads();
  const bool group_over = s_over != 0;
  if (ot.active && lane == 0) a.info[dir][tile] = group_over ? -1 : count;
  if (group_over && tid == 0) a.over[dir][atomicAdd(a.over_count[dir], 1)] = make_int4(g, 0, 0, 0);
}

// Byte offset of dims half `half` of token `id`'s row of head h in [T][H][16]
// bf16; list pads (id < 0) address past every resource and load zeros.
DEVI uint32_t list_row_off(int id, int H, int h, int half) {
  return id < 0 ? 0x80000000u : ((uint32_t)id * H + h) * (kHd * 2) + 16u * half;
}

// 0 if bit K of w is set, else -inf: v_bfe_i32 (the bit sign-extended to a
// full mask) and v_bfi_b32 (-inf where the mask is clear).  Written as asm:
// the compiler turns the C form into a compare and a select, three
// instructions and a VCC hazard per element.
template <int K>
DEVI float bit_bias(uint32_t w, int ninf) {
  float b;
  asm("v_bfe_i32 %0, %1, %2, 1\n\tv_bfi_b32 %0, %0, 0, %3" : "=&v"(b) : "v"(w), "i"(K), "s"(ninf));
  return b;
}
template <int R>
DEVI void word_bias_rows(f32x16& b, uint32_t w, int ninf) {
  if constexpr (R < 16) {
    b[R] = bit_bias<16 * (R >> 3) + (R & 7)>(w, ninf);
    word_bias_rows<R + 1>(b, w, ninf);
  }
}

// Bias (0 keep / -inf drop) of the lane's 16 accumulator rows (tile-local
// partner row_local(r, half)) from its mask word.
DEVI f32x16 word_bias(uint32_t w, int half) {
  f32x16 b;
  word_bias_rows<0>(b, w >> (8 * half), (int)0xff800000);
  return b;
}

// x of lane l ^ 32 combined with x by op (sum, max): v_permlane32_swap.
DEVI float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}
DEVI float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}

// XCD-aware block order.  Blocks go to the 8 XCDs round-robin (block b on
// XCD b % 8), each XCD with its own L2.  Work item i of n (group-major:
// i = group * head groups + head group) runs on block (i % per) * 8 + i / per,
// per = ceil(n / 8): XCD x takes items [x per, (x + 1) per) in order, a
// contiguous token range over all heads, so the partner rows its waves gather
// (whole 512-byte token rows over the heads) are shared in its L2.  Returns
// -1 for the grid's spare blocks.
#ifndef ESA_LIST_XCD
#define ESA_LIST_XCD 1
#endif
constexpr int kXcds = 8;
DEVI int list_item(int n_items) {
  if (!ESA_LIST_XCD) return (int)blockIdx.x < n_items ? (int)blockIdx.x : -1;
  const int per = (n_items + kXcds - 1) / kXcds;
  const int i = (int)(blockIdx.x % kXcds) * per + (int)(blockIdx.x / kXcds);
  return i < n_items ? i : -1;
}

static_assert(kListCap >= 128, "list_tile reads the first 128 ids");

#ifndef ESA_LIST_HEADS
#define ESA_LIST_HEADS 2
#endif
#ifndef ESA_LIST_HEADS_KV
#define ESA_LIST_HEADS_KV 2
#endif
constexpr int kListHeads = ESA_LIST_HEADS;       // heads per wave of the forward and dQ list kernels
constexpr int kListHeadsKv = ESA_LIST_HEADS_KV;  // heads per wave of the dK/dV list kernel

template <int NH>
struct StageList { i32x4 k[NH], v[NH]; uint32_t w; };


// ---- LDS-direct staging of the list kernels (dma16 / dma4 / wait_vmcnt:
// esa_attn_tiles.h)
// kDmaDepth stage buffers: stage s is staged in buffer s % kDmaDepth while
// the next kDmaDepth - 1 stages are in flight.  issue(stage, buf) issues a
// stage's loads (kPer of them); past the last stage it re-issues the last one
// into a spare buffer, so every wait covers exactly kDmaDepth - 1 stages of
// later loads.  A stage's buffer is reloaded only after the stage's compute
// has consumed its reads.
#ifndef ESA_DMA_DEPTH
#define ESA_DMA_DEPTH 2
#endif
constexpr int kDmaDepth = ESA_DMA_DEPTH;
static_assert(kDmaDepth >= 2 && kDmaDepth <= 4, "stage buffers");
template <int kPer, class Issue, class Compute>
DEVI void dma_pipeline(int n, Issue issue, Compute compute) {
  if (n <= 0) return;
#pragma unroll
  for (int i = 0; i < kDmaDepth - 1; ++i) issue(min(i, n - 1), i);
  int buf = 0, nxt = kDmaDepth - 1;   // st % kDmaDepth, (st + kDmaDepth - 1) % kDmaDepth
  for (int st = 0; st < n; ++st) {
    issue(min(st + kDmaDepth - 1, n - 1), nxt);
    wait_vmcnt<(kDmaDepth - 1) * kPer>();
    wave_sync();
    compute(st, buf);
    buf = buf == kDmaDepth - 1 ? 0 : buf + 1;
    nxt = nxt == kDmaDepth - 1 ? 0 : nxt + 1;
  }
  wait_vmcnt<0>();   // the re-issued loads land before the wave's LDS can be reallocated
}

// Blocks of the list kernels: one 32-token tile and kWaves head groups (one
// per wave).  The waves gather complementary slices of the same partner rows
// ([T][H][16] bf16: a token's heads are contiguous), so the cache lines they
// pull are shared in the CU's L1 instead of each CU using a fraction of every
// line; the tile's ids are loaded once per block.
DEVI int list_block_ids(const AttnArgs& a, int tile, int* sid, int tid) {
  const int n = a.info[tile];
  if (n > 0) {
    const int* ids = a.ids + (size_t)tile * kListCap;
    const int m = (n + kTile - 1) & ~(kTile - 1);
    for (int i = tid; i < m; i += 256) sid[i] = ids[i];
  }
  __syncthreads();
  return n < 0 ? -1 : (n + kTile - 1) / kTile;
}

// Forward over the key lists: one wave = one 32-query tile and kListHeads
// heads; the bias of a compact tile seeds every head's score MFMA; online
// softmax (running max per query, rescaled when it grows).
__global__ __launch_bounds__(256) void list_fwd_kernel(const AttnArgs a) {
  constexpr int NH = kListHeads;
  __shared__ __align__(16) bf16 sK[kWaves][kDmaDepth][NH][2 * kTileHalf];   // K rows split by dims half
  __shared__ __align__(16) bf16 sV[kWaves][kDmaDepth][NH][2 * kTileHalf];   // V rows split by dims half
  __shared__ __align__(16) uint32_t sW[kWaves][kDmaDepth][64];               // mask words (lane col)
  __shared__ int sId[kListCap];
  __shared__ __align__(16) bf16 sOnes[4];                                    // the ones rows of [V^T ; 1]
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5, c16 = lane & 15, grp = lane >> 4;
  const int H = a.heads, n_hg = (H + NH - 1) / NH, n_hq = (n_hg + kWaves - 1) / kWaves;
  const int idx = list_item(((a.total_q + kTile - 1) / kTile) * n_hq);
  if (idx < 0) return;
  const int tile = idx / n_hq, hg = (idx - tile * n_hq) * kWaves + wave;
  const int h0 = hg * NH, nh = min(NH, H - h0);   // nh <= 0: a wave without heads
  if (tid < 4) sOnes[tid] = (bf16)1.f;
  const int oi = tile * kTile + col;
  const bool valid = oi < a.total_q;
  const int oc = valid ? oi : a.total_q - 1;
  bf16x8 qf[NH];
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    const int hc = min(max(h0, 0) + u, H - 1);
    qf[u] = *reinterpret_cast<const bf16x8*>(a.q + ((size_t)oc * H + hc) * kHd + 8 * half);
  }
  const int nct = list_block_ids(a, tile, sId, tid);   // no partners: acc stays 0, rows 0, lse -inf
  if (nct < 0 || nh <= 0) return;
  bf16x8 qh[NH], ql[NH];
  float m_run[NH];
  f32x16 acc[NH];
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    split_scaled(qf[u], a.c, qh[u], ql[u]);
    m_run[u] = -INFINITY;
    acc[u] = f32x16{};
  }
  const uint32_t kv_bytes = (uint32_t)a.total_k * H * kHd * 2;
  const rsrc_t rk = make_rsrc(a.k, kv_bytes), rv = make_rsrc(a.v, kv_bytes);
  const rsrc_t rw = make_rsrc(a.bits + (size_t)tile * kListCap, (uint32_t)kListCap * 4u);
  dma_pipeline<2 * NH + 1>(
      nct,
      [&](int c, int buf) {
        const int id = sId[c * kTile + col];
#pragma unroll
        for (int u = 0; u < NH; ++u) {
          const uint32_t off = list_row_off(id, H, min(h0 + u, H - 1), half);
          dma16(rk, off, sK[wave][buf][u]);
          dma16(rv, off, sV[wave][buf][u]);
        }
        dma4(rw, (uint32_t)(c * kTile + col) * 4u, sW[wave][buf]);
      },
      [&](int, int buf) {
        const f32x16 bias = word_bias(sW[wave][buf][col], half);
#pragma unroll
        for (int u = 0; u < NH; ++u) {
          if (u >= nh) break;   // wave-uniform
          const bf16x8 kr = half_row8<kTileHalf>(sK[wave][buf][u], kperm(col), half);
          const f32x16 s = mfma32(kr, ql[u], mfma32(kr, qh[u], bias));
          float mt = s[0];
#pragma unroll
          for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
          mt = halves_max(mt);
          const float m_new = fmaxf(m_run[u], mt);
          if (__ballot(m_new > m_run[u])) {
            const float alpha = fast_exp2(m_run[u] - (m_new == -INFINITY ? 0.f : m_new));
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[u][r] *= alpha;
            m_run[u] = m_new;
          }
          const float m_use = m_run[u] == -INFINITY ? 0.f : m_run[u];
          float p[16];
#pragma unroll
          for (int r = 0; r < 16; ++r) p[r] = fast_exp2(s[r] - m_use);
          bf16x8 vt0, vt1;
          tr_rows32<kTileHalf>(sV[wave][buf][u], 0, sOnes, c16, grp, vt0, vt1);
          acc[u] = mfma32(vt0, cvt8(p), acc[u]);
          acc[u] = mfma32(vt1, cvt8(p + 8), acc[u]);
        }
      });
  if (!valid) return;
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    if (u >= nh) break;
    const int h = h0 + u;
    const float l = acc[u][8];   // a ones row of [V^T; 1] P^T: the softmax row sum
    store_rows8(a.o + ((size_t)oi * H + h) * kHd, acc[u], l > 0.f ? 1.f / l : 0.f, half);
    if (half == 0)
      a.lse_out[(size_t)h * a.total_q + oi] = l > 0.f ? (m_run[u] + fast_log2(l)) * kLn2 : -INFINITY;
  }
}

// dQ over the key lists: one wave = one 32-query tile and kListHeads heads,
// blocks and staging as the forward.  Each wave also writes its heads' row
// statistics of the dK/dV pass (every tile, also those the walk kernels take).
__global__ __launch_bounds__(256) void list_dq_kernel(const AttnArgs a) {
  constexpr int NH = kListHeads;
  __shared__ __align__(16) bf16 sK[kWaves][kDmaDepth][NH][2 * kTileHalf];   // K rows split by dims half
  __shared__ __align__(16) bf16 sV[kWaves][kDmaDepth][NH][2 * kTileHalf];   // V rows split by dims half
  __shared__ __align__(16) uint32_t sW[kWaves][kDmaDepth][64];               // mask words (lane col)
  __shared__ int sId[kListCap];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5, c16 = lane & 15, grp = lane >> 4;
  const int H = a.heads, n_hg = (H + NH - 1) / NH, n_hq = (n_hg + kWaves - 1) / kWaves;
  const int idx = list_item(((a.total_q + kTile - 1) / kTile) * n_hq);
  if (idx < 0) return;
  const int tile = idx / n_hq, hg = (idx - tile * n_hq) * kWaves + wave;
  const int h0 = hg * NH, nh = min(NH, H - h0);   // nh <= 0: a wave without heads
  const int oi = tile * kTile + col;
  const bool valid = oi < a.total_q;
  const int oc = valid ? oi : a.total_q - 1;
  bf16x8 qf[NH], dof[NH], of[NH];
  float lq[NH];
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    const int hc = min(max(h0, 0) + u, H - 1);
    const size_t row = ((size_t)oc * H + hc) * kHd + 8 * half;
    qf[u] = *reinterpret_cast<const bf16x8*>(a.q + row);
    dof[u] = *reinterpret_cast<const bf16x8*>(a.dout + row);
    of[u] = *reinterpret_cast<const bf16x8*>(a.out + row);
    lq[u] = a.lse[(size_t)hc * a.total_q + oc];
  }
  float dsum[NH], lse2q[NH];
  f32x16 acc[NH];
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) d = fmaf((float)dof[u][e], (float)of[u][e], d);
    dsum[u] = halves_sum(d);
    lse2q[u] = lq[u] == -INFINITY ? INFINITY : lq[u] * kLog2e;
    acc[u] = f32x16{};
    // Row statistics of the dK/dV pass, as bf16 (hi, lo) pairs: -LSE2/c (-1e30
    // for rows without keys and padding: their P is 0) and -D.
    if (half == 0 && u < nh) {
      const float xs = valid && lq[u] != -INFINITY ? -(lq[u] * kLog2e) / a.c : kDeadRow;
      a.aux_out[(size_t)(h0 + u) * a.tq_pad + oi] =
          make_uint2(split_bf16_pair(xs), split_bf16_pair(valid ? -dsum[u] : 0.f));
    }
  }
  const int nct = list_block_ids(a, tile, sId, tid);
  if (nct < 0 || nh <= 0) return;
  const f32x16 zero = {};
  const uint32_t kv_bytes = (uint32_t)a.total_k * H * kHd * 2;
  const rsrc_t rk = make_rsrc(a.k, kv_bytes), rv = make_rsrc(a.v, kv_bytes);
  const rsrc_t rw = make_rsrc(a.bits + (size_t)tile * kListCap, (uint32_t)kListCap * 4u);
  dma_pipeline<2 * NH + 1>(
      nct,
      [&](int c, int buf) {
        const int id = sId[c * kTile + col];
#pragma unroll
        for (int u = 0; u < NH; ++u) {
          const uint32_t off = list_row_off(id, H, min(h0 + u, H - 1), half);
          dma16(rk, off, sK[wave][buf][u]);
          dma16(rv, off, sV[wave][buf][u]);
        }
        dma4(rw, (uint32_t)(c * kTile + col) * 4u, sW[wave][buf]);
      },
      [&](int, int buf) {
        const f32x16 bias = word_bias(sW[wave][buf][col], half);
#pragma unroll
        for (int u = 0; u < NH; ++u) {
          if (u >= nh) break;   // wave-uniform
          const f32x16 s = mfma32(half_row8<kTileHalf>(sK[wave][buf][u], kperm(col), half), qf[u], bias);
          const f32x16 dp = mfma32(half_row8<kTileHalf>(sV[wave][buf][u], kperm(col), half), dof[u], zero);
          float ds[16];
#pragma unroll
          for (int r = 0; r < 16; ++r) ds[r] = fast_exp2(fmaf(s[r], a.c, -lse2q[u])) * (dp[r] - dsum[u]);
          bf16x8 kt0, kt1;
          tr_rows32<kTileHalf>(sK[wave][buf][u], 0, nullptr, c16, grp, kt0, kt1);
          acc[u] = mfma32(kt0, cvt8(ds), acc[u]);
          acc[u] = mfma32(kt1, cvt8(ds + 8), acc[u]);
        }
      });
  if (!valid) return;
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    if (u >= nh) break;
    store_rows8(a.dq + ((size_t)oi * H + h0 + u) * kHd, acc[u], a.scale, half);
  }
}

// dK/dV over the key lists (of the key tiles, or of the query tiles when the
// mask is symmetric): one wave = one 32-key tile and kListHeadsKv heads,
// blocks and staging as the forward.  A stage gathers the partner queries'
// Q and dO rows and their row statistics (per two heads, the records'
// two words in [2][64] arrays: lanes of half j carry head 2 i + j).
__global__ __launch_bounds__(256) void list_dkdv_kernel(const AttnArgs a0) {
  AttnArgs a = a0;
  if (!*a0.sym) {   // the key tiles' own lists
    a.info = a0.kinfo;
    a.ids = a0.kids;
    a.bits = a0.kbits;
  }
  constexpr int NH = kListHeadsKv;
  constexpr int NA = (NH + 1) / 2;   // row-statistic record pairs per stage
  __shared__ __align__(16) bf16 sQ[kWaves][kDmaDepth][NH][2 * kTileHalf];    // Q rows split by dims half
  __shared__ __align__(16) bf16 sDO[kWaves][kDmaDepth][NH][2 * kTileHalf];   // dO rows split by dims half
  __shared__ __align__(16) uint32_t sAux[kWaves][kDmaDepth][NA][2][64];     // row-statistic MFMA operands
  __shared__ __align__(16) uint32_t sW[kWaves][kDmaDepth][64];               // mask words (lane col)
  __shared__ int sId[kListCap];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5, c16 = lane & 15, grp = lane >> 4;
  const int H = a.heads, n_hg = (H + NH - 1) / NH, n_hq = (n_hg + kWaves - 1) / kWaves;
  const int idx = list_item(((a.total_k + kTile - 1) / kTile) * n_hq);
  if (idx < 0) return;
  const int tile = idx / n_hq, hg = (idx - tile * n_hq) * kWaves + wave;
  const int h0 = hg * NH, nh = min(NH, H - h0);   // nh <= 0: a wave without heads
  const int oi = tile * kTile + col;
  const bool valid = oi < a.total_k;
  const int oc = valid ? oi : a.total_k - 1;
  bf16x8 kf[NH], vf[NH];
  f32x16 dva[NH], dka[NH];
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    const size_t row = ((size_t)oc * H + min(max(h0, 0) + u, H - 1)) * kHd + 8 * half;
    kf[u] = *reinterpret_cast<const bf16x8*>(a.k + row);
    vf[u] = *reinterpret_cast<const bf16x8*>(a.v + row);
    dva[u] = dka[u] = f32x16{};
  }
  const int nct = list_block_ids(a, tile, sId, tid);
  if (nct < 0 || nh <= 0) return;
  // B operand of the row-statistic MFMAs: ones in slots 0 and 1 (half 0).
  bf16x8 ones2 = {};
  if (half == 0) { ones2[0] = (bf16)1.f; ones2[1] = (bf16)1.f; }
  const f32x16 zero = {};
  const uint32_t q_bytes = (uint32_t)a.total_q * H * kHd * 2;
  const rsrc_t rq = make_rsrc(a.q, q_bytes), rd = make_rsrc(a.dout, q_bytes);
  const rsrc_t rx = make_rsrc(a.aux, (uint32_t)H * a.tq_pad * 8u);
  const rsrc_t rw = make_rsrc(a.bits + (size_t)tile * kListCap, (uint32_t)kListCap * 4u);
  dma_pipeline<2 * NH + 2 * NA + 1>(
      nct,
      [&](int c, int buf) {
        const int id = sId[c * kTile + col];
#pragma unroll
        for (int u = 0; u < NH; ++u) {
          const uint32_t off = list_row_off(id, H, min(h0 + u, H - 1), half);
          dma16(rq, off, sQ[wave][buf][u]);
          dma16(rd, off, sDO[wave][buf][u]);
        }
#pragma unroll
        for (int i = 0; i < NA; ++i) {
          const int hc = min(h0 + 2 * i + half, H - 1);
          const uint32_t off = id < 0 ? 0x80000000u : ((uint32_t)hc * a.tq_pad + id) * 8u;
          dma4(rx, off, sAux[wave][buf][i][0]);
          dma4(rx, off + 4u, sAux[wave][buf][i][1]);
        }
        dma4(rw, (uint32_t)(c * kTile + col) * 4u, sW[wave][buf]);
      },
      [&](int, int buf) {
        const f32x16 bias = word_bias(sW[wave][buf][col], half);
#pragma unroll
        for (int u = 0; u < NH; ++u) {
          if (u >= nh) break;   // wave-uniform
          const int ar = (u & 1) * kTile + kperm(col);
          const bf16x8 aux_s = as_bf16x8(i32x4{(int)sAux[wave][buf][u >> 1][0][ar], 0, 0, 0});
          const bf16x8 aux_d = as_bf16x8(i32x4{(int)sAux[wave][buf][u >> 1][1][ar], 0, 0, 0});
          // S' = Q K^T - LSE2/c + bias and dP' = dO V^T - D, rows = queries, lanes = keys.
          const f32x16 s =
              mfma32(half_row8<kTileHalf>(sQ[wave][buf][u], kperm(col), half), kf[u], mfma32(aux_s, ones2, bias));
          const f32x16 dp =
              mfma32(half_row8<kTileHalf>(sDO[wave][buf][u], kperm(col), half), vf[u], mfma32(aux_d, ones2, zero));
          float p[16], ds[16];
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            p[r] = fast_exp2(s[r] * a.c);
            ds[r] = p[r] * dp[r];
          }
          bf16x8 d0, d1, q0t, q1t;
          tr_rows32<kTileHalf>(sDO[wave][buf][u], 0, nullptr, c16, grp, d0, d1);
          tr_rows32<kTileHalf>(sQ[wave][buf][u], 0, nullptr, c16, grp, q0t, q1t);
          dva[u] = mfma32(d0, cvt8(p), dva[u]);
          dva[u] = mfma32(d1, cvt8(p + 8), dva[u]);
          dka[u] = mfma32(q0t, cvt8(ds), dka[u]);
          dka[u] = mfma32(q1t, cvt8(ds + 8), dka[u]);
        }
      });
  if (!valid) return;
#pragma unroll
  for (int u = 0; u < NH; ++u) {
    if (u >= nh) break;
    const int h = h0 + u;
    store_rows8(a.dv + ((size_t)oi * H + h) * kHd, dva[u], 1.f, half);
    store_rows8(a.dk + ((size_t)oi * H + h) * kHd, dka[u], a.scale, half);
  }
}

// ======================================================================== fp32 path
// fp32 q, k, v, outputs and softmax (the reference's fp32 modules, compared
// at 1e-5 relative).  One thread per (outer token, head) of a group of up to
// 128 outer tokens of one segment (a per-segment plan, longest partner range
// first: a block walks only its own segment's partners, so few-query
// segments such as PMA seeds get one block per segment and head), partner
// runs of 32 tokens staged in LDS and read by broadcast (the forward holds a
// partner row across each 16-lane wave row instead and splits a group's key
// tiles over several thread groups; see attn_fwd_f32_kernel).  Scores,
// softmax and both products are fp32 FMA chains in a fixed order.  Exponentials and the
// log-sum-exp use the hardware v_exp_f32 / v_log_f32 (about 1 ulp): every
// exponent is <= 0 (a score minus the running maximum or the row's LSE2) and
// every log argument >= 1 (the row sum includes the maximum's 1), so the
// flushed denormal results of the hardware ops are below 2^-126 of the
// row's weights.  With attention dropout (DROP, unmasked calls) the staged
// partner tile carries the partners' keys of the keep mask (esa_common.h):
// a dropped partner's probability leaves the products over partners and its
// dP leaves dS; outputs carry 1 / (1 - p).

struct AttnF32Args {
  DropoutCfg drop;
  const float* q; const float* k; const float* v; const float* out; const float* dout;
  const float2* rows;       // backward: per (head, query) (LSE2 or +inf for rows without keys, D) [H][tq_pad]
  int total_q, total_k, heads, tq_pad;
  float c, scale;           // c = softmax_scale * log2(e)
  const int2* nodes;        // edge mask: per-token node pairs (padded)
  const int4* plan;         // (outer begin, outer segment end, partner begin, partner end) per group
  const int* count;         // number of groups
  float* o; float* lse_out; float* dq; float* dk; float* dv;
};

constexpr int kF32Threads = kGroupTok;

// Rows of HD fp32 values (HD = 16, 24, 32 or 64) as float4 chunks.
template <int HD>
DEVI void loadn(const float* p, float x[HD]) {
#pragma unroll
  for (int i = 0; i < HD / 4; ++i) {
    const float4 v = reinterpret_cast<const float4*>(p)[i];
    x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
  }
}
template <int HD>
DEVI void storen(float* p, const float x[HD], float mul) {
#pragma unroll
  for (int i = 0; i < HD / 4; ++i)
    reinterpret_cast<float4*>(p)[i] = make_float4(x[4 * i] * mul, x[4 * i + 1] * mul, x[4 * i + 2] * mul,
                                                  x[4 * i + 3] * mul);
}
template <int HD>
DEVI float dotn(const float x[HD], const float4* y) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < HD / 4; ++i) {
    const float4 v = y[i];
    s = fmaf(x[4 * i], v.x, s); s = fmaf(x[4 * i + 1], v.y, s);
    s = fmaf(x[4 * i + 2], v.z, s); s = fmaf(x[4 * i + 3], v.w, s);
  }
  return s;
}
template <int HD>
DEVI void axpyn(float a, const float4* y, float x[HD]) {
#pragma unroll
  for (int i = 0; i < HD / 4; ++i) {
    const float4 v = y[i];
    x[4 * i] = fmaf(a, v.x, x[4 * i]); x[4 * i + 1] = fmaf(a, v.y, x[4 * i + 1]);
    x[4 * i + 2] = fmaf(a, v.z, x[4 * i + 2]); x[4 * i + 3] = fmaf(a, v.w, x[4 * i + 3]);
  }
}

// Stage the 32 tokens from t0 of a [T][H][HD] fp32 tensor into LDS [32][HD / 4]
// float4 (128 threads, HD / 16 float4 each); tokens at or past `end` read as zeros.
template <int HD>
DEVI void stage_rows_f32(float4 (*dst)[HD / 4], const float* src, int end, int H, int head, int t0, int tid) {
#pragma unroll
  for (int i = tid; i < kTile * HD / 4; i += kF32Threads) {
    const int t = t0 + i / (HD / 4), part = i % (HD / 4);
    dst[i / (HD / 4)][part] = t < end ? reinterpret_cast<const float4*>(src + ((size_t)t * H + head) * HD)[part]
                                      : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// Admissible partner p (below the segment's partner end phi) of outer token oi.
template <bool MASKED>
DEVI bool admissible_f32(int p, int phi, int oi, int2 pn, int2 own) {
  bool ok = p < phi;
  if (MASKED) ok = ok && p != oi && node_adjacent(pn, own);
  return ok;
}

// This thread's outer token of group g (clamped into the group when past its
// segment's end).
struct F32Outer { int oi, oc; bool valid; int plo, phi; };
DEVI F32Outer f32_outer(const int4& g, int tid) {
  F32Outer o;
  o.oi = g.x + tid;
  o.valid = o.oi < g.y;
  o.oc = o.valid ? o.oi : g.x;
  o.plo = g.z;
  o.phi = g.w;
  return o;
}

// Partner rows across a wave row.  A staged partner row of HD fp32 values is
// held by the 16 lanes of each wave row: lane l holds dims l % 16,
// 16 + l % 16, ... (NR = ceil(HD / 16) registers, zeros past HD), and all
// four rows of the wave hold the same partner.  `v_fmac_f32_dpp` with
// row_newbcast:i hands dim 16 r + i of that partner to the 16 lanes of each
// row inside the multiply-add, so a product with a partner row costs one VALU
// instruction per dim and one 4-byte LDS read per partner and lane.  Read as
// whole rows per lane, the same partner costs HD / 4 16-byte reads per lane:
// the broadcast reads move 64 x 16 bytes through the LDS pipe each, and they,
// not the FMAs, bounded the kernels.  DPP reads the source lane's register,
// so every lane of the wave is active at these instructions (lanes past
// their group's end compute on a clamped token and store nothing).  The
// leading s_nop 1 covers the two wait states a DPP read of a VGPR needs
// after a VALU write of it.
#define F32_FM(ACC, SRC, MUL, I) \
  "v_fmac_f32_dpp %" #ACC ", %" #SRC ", %" #MUL " row_newbcast:" #I " row_mask:0xf bank_mask:0xf\n\t"
#define F32_DOT4(I, Q) F32_FM(0, 4, Q, I) F32_FM(1, 5, Q, I) F32_FM(2, 6, Q, I) F32_FM(3, 7, Q, I)
#define F32_AXPY8(V, P)                                                                                 \
  F32_FM(0, V, P, 0) F32_FM(1, V, P, 1) F32_FM(2, V, P, 2) F32_FM(3, V, P, 3) F32_FM(4, V, P, 4)         \
  F32_FM(5, V, P, 5) F32_FM(6, V, P, 6) F32_FM(7, V, P, 7)
#define F32_AXPY16(V, P)                                                                                \
  F32_AXPY8(V, P) F32_FM(8, V, P, 8) F32_FM(9, V, P, 9) F32_FM(10, V, P, 10) F32_FM(11, V, P, 11)        \
  F32_FM(12, V, P, 12) F32_FM(13, V, P, 13) F32_FM(14, V, P, 14) F32_FM(15, V, P, 15)

// s[k] += sum over the register's N dims (8 or 16, ascending) of x[i] * dim i
// of partner k's row register y[k], for four partners.
template <int N>
DEVI void dot4_rows(float (&s)[4], const float (&y)[4], const float* x) {
  if constexpr (N == 16)
    asm("s_nop 1\n\t"
        F32_DOT4(0, 8) F32_DOT4(1, 9) F32_DOT4(2, 10) F32_DOT4(3, 11) F32_DOT4(4, 12) F32_DOT4(5, 13)
        F32_DOT4(6, 14) F32_DOT4(7, 15) F32_DOT4(8, 16) F32_DOT4(9, 17) F32_DOT4(10, 18) F32_DOT4(11, 19)
        F32_DOT4(12, 20) F32_DOT4(13, 21) F32_DOT4(14, 22) F32_DOT4(15, 23)
        : "+v"(s[0]), "+v"(s[1]), "+v"(s[2]), "+v"(s[3])
        : "v"(y[0]), "v"(y[1]), "v"(y[2]), "v"(y[3]), "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]),
          "v"(x[5]), "v"(x[6]), "v"(x[7]), "v"(x[8]), "v"(x[9]), "v"(x[10]), "v"(x[11]), "v"(x[12]),
          "v"(x[13]), "v"(x[14]), "v"(x[15]));
  else
    asm("s_nop 1\n\t"
        F32_DOT4(0, 8) F32_DOT4(1, 9) F32_DOT4(2, 10) F32_DOT4(3, 11) F32_DOT4(4, 12) F32_DOT4(5, 13)
        F32_DOT4(6, 14) F32_DOT4(7, 15)
        : "+v"(s[0]), "+v"(s[1]), "+v"(s[2]), "+v"(s[3])
        : "v"(y[0]), "v"(y[1]), "v"(y[2]), "v"(y[3]), "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]),
          "v"(x[5]), "v"(x[6]), "v"(x[7]));
}

// x[i] += a * dim i of the row register y, over the register's N dims (8 or 16).
template <int N>
DEVI void axpy_row(float* x, float y, float a) {
  if constexpr (N == 16)
    asm("s_nop 1\n\t" F32_AXPY16(16, 17)
        : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]), "+v"(x[7]),
          "+v"(x[8]), "+v"(x[9]), "+v"(x[10]), "+v"(x[11]), "+v"(x[12]), "+v"(x[13]), "+v"(x[14]), "+v"(x[15])
        : "v"(y), "v"(a));
  else
    asm("s_nop 1\n\t" F32_AXPY8(8, 9)
        : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]), "+v"(x[7])
        : "v"(y), "v"(a));
}

// Dims held by register r of an HD-wide row (16, or 8 for the last register of HD 24).
template <int HD>
DEVI constexpr int row_dims(int r) { return HD - 16 * r >= 16 ? 16 : HD - 16 * r; }

// A partner row's registers for lane li: y[r] = dim 16 r + li of the row.
template <int HD>
DEVI void row_regs(float (&y)[(HD + 15) / 16], const float* row, int li) {
#pragma unroll
  for (int r = 0; r < (HD + 15) / 16; ++r) y[r] = row[16 * r + li];
}

// Four partners' dot products with the lane's row x (HD dims, ascending):
// s[k] = sum_d x[d] * dim d of partner k, from the partners' row registers.
template <int HD, int R = 0>
DEVI void dot4(float (&s)[4], const float* x, const float (&y)[4][(HD + 15) / 16]) {
  if constexpr (R == 0) s[0] = s[1] = s[2] = s[3] = 0.f;
  if constexpr (16 * R < HD) {
    const float yr[4] = {y[0][R], y[1][R], y[2][R], y[3][R]};
    dot4_rows<row_dims<HD>(R)>(s, yr, x + 16 * R);
    dot4<HD, R + 1>(s, x, y);
  }
}

// x[d] += a * dim d of a partner row (HD dims) from its row registers.
template <int HD, int R = 0>
DEVI void axpy(float* x, float a, const float (&y)[(HD + 15) / 16]) {
  if constexpr (16 * R < HD) {
    axpy_row<row_dims<HD>(R)>(x + 16 * R, y[R], a);
    axpy<HD, R + 1>(x, a, y);
  }
}

// Stage the 32 tokens from t0 of a [T][H][HD] fp32 tensor into LDS rows of
// 16 NR floats (128 threads): dims past HD and tokens at or past `end` are zeros.
template <int HD>
DEVI void stage_rows_lane(float (*dst)[16 * ((HD + 15) / 16)], const float* src, int end, int H, int head, int t0,
                          int tid) {
  constexpr int C = 4 * ((HD + 15) / 16);   // float4 chunks per staged row
#pragma unroll
  for (int i = tid; i < kTile * C; i += kF32Threads) {
    const int t = t0 + i / C, part = i % C;
    reinterpret_cast<float4*>(dst[i / C])[part] =
        t < end && part < HD / 4 ? reinterpret_cast<const float4*>(src + ((size_t)t * H + head) * HD)[part]
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// Key splits of the fp32 forward: S groups of 128 threads per block take the
// group's key tiles in turn (tile i goes to split i mod S), each with its own
// staging buffers, and merge their (max, sum, output) partials at the end in
// split order.  One thread per (query, head) gives only a few thousand waves
// per call (configuration 0: 2,392 for 1,024 SIMDs) with per-block work
// proportional to the segment length; with the splits the long segments'
// blocks finish S times sooner and the SIMDs hold S times the waves.
template <int HD>
constexpr int f32_splits() { return HD >= 64 ? 2 : 4; }

template <bool MASKED, int HD, bool DROP>
__global__ __launch_bounds__(kF32Threads * f32_splits<HD>()) void attn_fwd_f32_kernel(const AttnF32Args a) {
  constexpr int NR = (HD + 15) / 16, S = f32_splits<HD>();
  __shared__ float sK[S][kTile][16 * NR], sV[S][kTile][16 * NR];
  __shared__ int2 sN[S][kTile];
  __shared__ uint32_t sKey[S][DROP ? kTile : 1];   // column keys of the staged keys
  __shared__ float sAcc[kF32Threads][16 * NR + 1];   // a later split's partial: output row, then m and l
  __shared__ float sML[kF32Threads][2];
  const int split = threadIdx.x / kF32Threads, tid = threadIdx.x - split * kF32Threads, li = tid & 15;
  const int H = a.heads;
  const int item = blockIdx.x / H, head = blockIdx.x - item * H;
  if (item >= *a.count) return;
  const F32Outer ot = f32_outer(a.plan[item], tid);
  const int oi = ot.oi, oc = ot.oc, phi = ot.phi;
  float q[16 * NR], acc[16 * NR];
  loadn<HD>(a.q + ((size_t)oc * H + head) * HD, q);
#pragma unroll
  for (int i = 0; i < 16 * NR; ++i) {
    if (i >= HD) q[i] = 0.f;
    acc[i] = 0.f;
  }
  const int2 own = MASKED ? a.nodes[oc] : make_int2(0, 0);
  const uint32_t rk = DROP ? drop_row(a.drop, oc, head) : 0u;
  float m = -INFINITY, l = 0.f;
  const int rounds = (phi - ot.plo + S * kTile - 1) / (S * kTile);
  for (int it = 0; it < rounds; ++it) {
    const int k0 = ot.plo + (it * S + split) * kTile;   // past phi: nothing to do this round (split-uniform)
    __syncthreads();
    if (k0 < phi) {
      stage_rows_lane<HD>(sK[split], a.k, phi, H, head, k0, tid);
      stage_rows_lane<HD>(sV[split], a.v, phi, H, head, k0, tid);
      if (MASKED && tid < kTile) sN[split][tid] = k0 + tid < phi ? a.nodes[k0 + tid] : make_int2(-1, -1);
      if (DROP && tid < kTile) sKey[split][tid] = drop_col(a.drop, k0 + tid);
    }
    __syncthreads();
    if (k0 >= phi) continue;
    float s[kTile];
    float mt = -INFINITY;
    float ky[kTile][NR];   // the tile's key rows, loaded one group of four ahead of their products
#pragma unroll
    for (int u = 0; u < 4; ++u) row_regs<HD>(ky[u], sK[split][u], li);
#pragma unroll
    for (int j = 0; j < kTile; j += 4) {
      if (j + 4 < kTile) {
#pragma unroll
        for (int u = 4; u < 8; ++u) row_regs<HD>(ky[j + u], sK[split][j + u], li);
      }
      __builtin_amdgcn_sched_barrier(0);   // keep the next group's reads ahead of these products
      float d[4];
      dot4<HD>(d, q, *reinterpret_cast<const float(*)[4][NR]>(&ky[j]));
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int2 pn = MASKED ? sN[split][j + u] : make_int2(0, 0);
        s[j + u] = admissible_f32<MASKED>(k0 + j + u, phi, oi, pn, own) ? a.c * d[u] : -INFINITY;
        mt = fmaxf(mt, s[j + u]);
      }
    }
    if (mt > m) {
      const float alpha = fast_exp2(m - mt);   // 0 while m = -inf
      l *= alpha;
#pragma unroll
      for (int i = 0; i < 16 * NR; ++i) acc[i] *= alpha;
      m = mt;
    }
    const float mb = m == -INFINITY ? 0.f : m;   // no admissible key yet: every p is exp2(-inf) = 0
    float vy[kTile][NR];   // value rows, loaded four keys ahead of their products
#pragma unroll
    for (int j = 0; j < 4; ++j) row_regs<HD>(vy[j], sV[split][j], li);
#pragma unroll
    for (int j = 0; j < kTile; ++j) {
      if (j + 4 < kTile) row_regs<HD>(vy[j + 4], sV[split][j + 4], li);
      __builtin_amdgcn_sched_barrier(0);   // keep the reads four keys ahead of their product
      const float p = fast_exp2(s[j] - mb);
      l += p;
      axpy<HD>(acc, DROP && !drop_keep(a.drop, rk, sKey[split][j], k0 + j) ? 0.f : p, vy[j]);
    }
  }
  // Merge in split order: split 0 takes over split 1's partial, then split 2's, ...
  // (m = -inf marks an empty partial; its output and sum are 0).
#pragma unroll
  for (int src = 1; src < S; ++src) {
    __syncthreads();
    if (split == src) {
#pragma unroll
      for (int i = 0; i < HD; ++i) sAcc[tid][i] = acc[i];
      sML[tid][0] = m;
      sML[tid][1] = l;
    }
    __syncthreads();
    if (split == 0) {
      const float m2 = sML[tid][0], l2 = sML[tid][1];
      const float mn = fmaxf(m, m2);
      if (mn != -INFINITY) {
        const float a1 = fast_exp2(m - mn), a2 = fast_exp2(m2 - mn);
        l = l * a1 + l2 * a2;
#pragma unroll
        for (int i = 0; i < HD; ++i) acc[i] = acc[i] * a1 + sAcc[tid][i] * a2;
        m = mn;
      }
    }
  }
  if (split != 0 || !ot.valid) return;
  storen<HD>(a.o + ((size_t)oi * H + head) * HD, acc, l > 0.f ? (DROP ? a.drop.inv_keep : 1.f) / l : 0.f);
  a.lse_out[(size_t)head * a.total_q + oi] = l > 0.f ? (m + fast_log2(l)) * kLn2 : -INFINITY;
}

// fp32 calls with segments of a few queries (the PMA's seeds: the expanded
// call has k queries per set).  The tiled fp32 kernels give each (segment,
// head) a 128-thread block in which k lanes are live and that walks every
// key of the segment, so their time is that of the longest segment's walk.
// Here the forward and dQ take one wave per (segment, query slot, head): its
// 64 lanes take the segment's keys in turn (key kb + lane + 64 i) with
// per-lane partials (running maximum and sum, or the dQ sum) that merge by a
// butterfly in a fixed order.  A slot also walks the segment's later queries
// (slot + slots, ...), so any number of queries per segment is computed; the
// caller's max_seqlen_q only sets the grid.  dK/dV takes one thread per (key,
// head) that walks its segment's queries.  (bf16 calls keep the MFMA
// kernels: with many heads and seeds, each slot's wave re-reading its
// segment's key rows costs more than the MFMA kernels' single pass.)
struct AttnFewArgs {
  DropoutCfg drop;
  const float* q; const float* k; const float* v; const float* out; const float* dout;
  const float* lse;
  const int* cu_q; const int* cu_k;
  int nseg, heads, total_q, total_k, slots, blocks_per_seg;
  float c, scale;
  float2* rows;   // backward: (LSE2, D) per (head, query), written by dQ, read by dK/dV; row stride total_q
  float* o; float* lse_out; float* dq; float* dk; float* dv;
};

// The wave's (segment, query slot, head) for the forward and dQ; false for a
// wave past the hint's slots (wave-uniform).
struct FewWave { int seg, slot, head; };
DEVI bool few_wave(const AttnFewArgs& a, FewWave& f) {
  f.seg = blockIdx.x / a.blocks_per_seg;
  const int w = (blockIdx.x - f.seg * a.blocks_per_seg) * 4 + (int)(threadIdx.x >> 6);
  f.slot = w / a.heads;
  f.head = w - f.slot * a.heads;
  return f.seg < a.nseg && f.slot < a.slots;
}

template <int HD, bool DROP>
__global__ __launch_bounds__(256) void attn_fwd_few_kernel(const AttnFewArgs a) {
  const int H = a.heads, lane = threadIdx.x & 63;
  FewWave f;
  if (!few_wave(a, f)) return;   // wave-uniform: no barriers in this kernel
  const int head = f.head;
  const int qb = a.cu_q[f.seg], qe = a.cu_q[f.seg + 1], kb = a.cu_k[f.seg], ke = a.cu_k[f.seg + 1];
  const float *Q = a.q, *K = a.k, *V = a.v;
  for (int qi = qb + f.slot; qi < qe; qi += a.slots) {
    float q[HD], acc[HD];
    loadn<HD>(Q + ((size_t)qi * H + head) * HD, q);
#pragma unroll
    for (int i = 0; i < HD; ++i) acc[i] = 0.f;
    const uint32_t rk = DROP ? drop_row(a.drop, qi, head) : 0u;
    float m = -INFINITY, l = 0.f;
    for (int kj = kb + lane; kj < ke; kj += 64) {
      float kx[HD];
      loadn<HD>(K + ((size_t)kj * H + head) * HD, kx);
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < HD; ++i) d = fmaf(q[i], kx[i], d);
      const float sc = a.c * d;
      if (sc > m) {
        const float alpha = fast_exp2(m - sc);   // 0 while m = -inf
        l *= alpha;
#pragma unroll
        for (int i = 0; i < HD; ++i) acc[i] *= alpha;
        m = sc;
      }
      const float p = fast_exp2(sc - m);
      l += p;
      const float pv = DROP && !drop_keep(a.drop, rk, drop_col(a.drop, kj), kj) ? 0.f : p;
      float vx[HD];
      loadn<HD>(V + ((size_t)kj * H + head) * HD, vx);
#pragma unroll
      for (int i = 0; i < HD; ++i) acc[i] = fmaf(pv, vx[i], acc[i]);
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {   // merge partials: max, rescaled sums and outputs
      const float m2 = __shfl_xor(m, off), l2 = __shfl_xor(l, off);
      const float mn = fmaxf(m, m2);
      const float a1 = mn == -INFINITY ? 0.f : fast_exp2(m - mn), a2 = mn == -INFINITY ? 0.f : fast_exp2(m2 - mn);
      l = l * a1 + l2 * a2;
#pragma unroll
      for (int i = 0; i < HD; ++i) {
        const float o2 = __shfl_xor(acc[i], off);
        acc[i] = acc[i] * a1 + o2 * a2;
      }
      m = mn;
    }
    if (lane == 0) {
      storen<HD>(a.o + ((size_t)qi * H + head) * HD, acc,
                       l > 0.f ? (DROP ? a.drop.inv_keep : 1.f) / l : 0.f);
      a.lse_out[(size_t)head * a.total_q + qi] = l > 0.f ? (m + fast_log2(l)) * kLn2 : -INFINITY;
    }
  }
}

// dQ_i = scale sum_j P_ij (dP_ij - D_i) k_j with P recomputed from the saved
// LSE and D_i = rowsum(dO_i * O_i); writes (LSE2, D) for the dK/dV pass.
template <int HD, bool DROP>
__global__ __launch_bounds__(256) void attn_dq_few_kernel(const AttnFewArgs a) {
  const int H = a.heads, lane = threadIdx.x & 63;
  FewWave f;
  if (!few_wave(a, f)) return;   // wave-uniform: no barriers in this kernel
  const int head = f.head;
  const int qb = a.cu_q[f.seg], qe = a.cu_q[f.seg + 1], kb = a.cu_k[f.seg], ke = a.cu_k[f.seg + 1];
  const float *Q = a.q, *K = a.k, *V = a.v;
  for (int qi = qb + f.slot; qi < qe; qi += a.slots) {
    float q[HD], g[HD], acc[HD];
    loadn<HD>(Q + ((size_t)qi * H + head) * HD, q);
    loadn<HD>(a.dout + ((size_t)qi * H + head) * HD, g);
    {
      float o[HD];
      loadn<HD>(a.out + ((size_t)qi * H + head) * HD, o);
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < HD; ++i) d = fmaf(g[i], o[i], d);
      acc[0] = d;   // D_i, the same in every lane
    }
    const float D = acc[0];
#pragma unroll
    for (int i = 0; i < HD; ++i) acc[i] = 0.f;
    const float lse = a.lse[(size_t)head * a.total_q + qi];
    const float lse2 = lse * kLog2e;   // a query without keys (-inf) walks no key
    const uint32_t rk = DROP ? drop_row(a.drop, qi, head) : 0u;
    for (int kj = kb + lane; kj < ke; kj += 64) {
      float kx[HD], vx[HD];
      loadn<HD>(K + ((size_t)kj * H + head) * HD, kx);
      loadn<HD>(V + ((size_t)kj * H + head) * HD, vx);
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int i = 0; i < HD; ++i) {
        s = fmaf(q[i], kx[i], s);
        dp = fmaf(g[i], vx[i], dp);
      }
      const float p = fast_exp2(a.c * s - lse2);
      if (DROP) dp = drop_keep(a.drop, rk, drop_col(a.drop, kj), kj) ? dp * a.drop.inv_keep : 0.f;
      const float ds = p * (dp - D);
#pragma unroll
      for (int i = 0; i < HD; ++i) acc[i] = fmaf(ds, kx[i], acc[i]);
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1)
#pragma unroll
      for (int i = 0; i < HD; ++i) acc[i] += __shfl_xor(acc[i], off);
    if (lane == 0) {
      storen<HD>(a.dq + ((size_t)qi * H + head) * HD, acc, a.scale);
      a.rows[(size_t)head * a.total_q + qi] = make_float2(lse2, D);
    }
  }
}

// dV_j = sum_i P_ij dO_i, dK_j = scale sum_i P_ij (dP_ij - D_i) q_i: one
// thread per (key, head), heads fastest; the key's segment by a binary search
// over cu_k; keys in no segment get zeros.
template <int HD, bool DROP>
__global__ __launch_bounds__(256) void attn_dkdv_few_kernel(const AttnFewArgs a) {
  const int H = a.heads;
  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long)a.total_k * H) return;
  const int kj = (int)(gid / H), head = (int)(gid - (long)kj * H);
  int lo = 0, hi = a.nseg;   // the last segment whose start is <= kj
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.cu_k[mid] <= kj) lo = mid; else hi = mid - 1;
  }
  const int seg = lo;
  float dk[HD], dv[HD];
#pragma unroll
  for (int i = 0; i < HD; ++i) dk[i] = dv[i] = 0.f;
  if (seg < a.nseg && kj >= a.cu_k[seg] && kj < a.cu_k[seg + 1]) {
    const int qb = a.cu_q[seg], qe = a.cu_q[seg + 1];
    float kx[HD], vx[HD];
    loadn<HD>(a.k + ((size_t)kj * H + head) * HD, kx);
    loadn<HD>(a.v + ((size_t)kj * H + head) * HD, vx);
    const uint32_t ck = DROP ? drop_col(a.drop, kj) : 0u;
    for (int qi = qb; qi < qe; ++qi) {
      float q[HD], g[HD];
      loadn<HD>(a.q + ((size_t)qi * H + head) * HD, q);
      loadn<HD>(a.dout + ((size_t)qi * H + head) * HD, g);
      const float2 rs = a.rows[(size_t)head * a.total_q + qi];
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int i = 0; i < HD; ++i) {
        s = fmaf(kx[i], q[i], s);
        dp = fmaf(vx[i], g[i], dp);
      }
      const float p = fast_exp2(a.c * s - rs.x);
      const bool keep = !DROP || drop_keep(a.drop, drop_row(a.drop, qi, head), ck, kj);
      const float pv = keep ? p : 0.f;
#pragma unroll
      for (int i = 0; i < HD; ++i) dv[i] = fmaf(pv, g[i], dv[i]);
      if (DROP) dp = keep ? dp * a.drop.inv_keep : 0.f;
      const float ds = p * (dp - rs.y);
#pragma unroll
      for (int i = 0; i < HD; ++i) dk[i] = fmaf(ds, q[i], dk[i]);
    }
  }
  storen<HD>(a.dv + ((size_t)kj * H + head) * HD, dv, DROP ? a.drop.inv_keep : 1.f);
  storen<HD>(a.dk + ((size_t)kj * H + head) * HD, dk, a.scale);
}

// dQ = scale * sum_j P_ij (dP_ij - D_i) k_j, P recomputed from the saved LSE.
template <bool MASKED, int HD, bool DROP>
__global__ __launch_bounds__(kF32Threads) void attn_dq_f32_kernel(const AttnF32Args a) {
  __shared__ float4 sK[kTile][HD / 4], sV[kTile][HD / 4];
  __shared__ int2 sN[kTile];
  __shared__ uint32_t sKey[DROP ? kTile : 1];   // column keys of the staged keys
  const int tid = threadIdx.x, H = a.heads;
  const int item = blockIdx.x / H, head = blockIdx.x - item * H;
  if (item >= *a.count) return;
  const F32Outer ot = f32_outer(a.plan[item], tid);
  const int oi = ot.oi, oc = ot.oc, phi = ot.phi;
  const bool valid = ot.valid;
  float q[HD], g[HD], acc[HD];
  loadn<HD>(a.q + ((size_t)oc * H + head) * HD, q);
  loadn<HD>(a.dout + ((size_t)oc * H + head) * HD, g);
#pragma unroll
  for (int i = 0; i < HD; ++i) acc[i] = 0.f;
  const float2 rs = a.rows[(size_t)head * a.tq_pad + oc];   // (LSE2, D)
  const int2 own = MASKED ? a.nodes[oc] : make_int2(0, 0);
  const uint32_t rk = DROP ? drop_row(a.drop, oc, head) : 0u;
  for (int k0 = ot.plo; k0 < phi; k0 += kTile) {
    __syncthreads();
    stage_rows_f32<HD>(sK, a.k, phi, H, head, k0, tid);
    stage_rows_f32<HD>(sV, a.v, phi, H, head, k0, tid);
    if (MASKED && tid < kTile) sN[tid] = k0 + tid < phi ? a.nodes[k0 + tid] : make_int2(-1, -1);
    if (DROP && tid < kTile) sKey[tid] = drop_col(a.drop, k0 + tid);
    __syncthreads();
    if (!valid) continue;
#pragma unroll
    for (int j = 0; j < kTile; ++j) {
      const int2 pn = MASKED ? sN[j] : make_int2(0, 0);
      if (!admissible_f32<MASKED>(k0 + j, phi, oi, pn, own)) continue;
      const float p = fast_exp2(a.c * dotn<HD>(q, sK[j]) - rs.x);
      float dp = dotn<HD>(g, sV[j]);
      if (DROP) dp = drop_keep(a.drop, rk, sKey[j], k0 + j) ? dp * a.drop.inv_keep : 0.f;
      const float ds = p * (dp - rs.y);
      axpyn<HD>(ds, sK[j], acc);
    }
  }
  if (!valid) return;
  storen<HD>(a.dq + ((size_t)oi * H + head) * HD, acc, a.scale);
}

// dV = sum_i P_ij dO_i, dK = scale * sum_i P_ij (dP_ij - D_i) q_i, one thread
// per key; the partner tiles are query tiles with their (LSE2, D).
template <bool MASKED, int HD, bool DROP>
__global__ __launch_bounds__(kF32Threads) void attn_dkdv_f32_kernel(const AttnF32Args a) {
  __shared__ float4 sQ[kTile][HD / 4], sG[kTile][HD / 4];
  __shared__ float2 sR[kTile];
  __shared__ int2 sN[kTile];
  __shared__ uint32_t sKey[DROP ? kTile : 1];   // row keys of the staged queries
  const int tid = threadIdx.x, H = a.heads;
  const int item = blockIdx.x / H, head = blockIdx.x - item * H;
  if (item >= *a.count) return;
  const F32Outer ot = f32_outer(a.plan[item], tid);
  const int oi = ot.oi, oc = ot.oc, phi = ot.phi;
  const bool valid = ot.valid;
  float kx[HD], vx[HD], dk[HD], dv[HD];
  loadn<HD>(a.k + ((size_t)oc * H + head) * HD, kx);
  loadn<HD>(a.v + ((size_t)oc * H + head) * HD, vx);
#pragma unroll
  for (int i = 0; i < HD; ++i) dk[i] = dv[i] = 0.f;
  const int2 own = MASKED ? a.nodes[oc] : make_int2(0, 0);
  const uint32_t ck = DROP ? drop_col(a.drop, oc) : 0u;
  for (int q0 = ot.plo; q0 < phi; q0 += kTile) {
    __syncthreads();
    stage_rows_f32<HD>(sQ, a.q, phi, H, head, q0, tid);
    stage_rows_f32<HD>(sG, a.dout, phi, H, head, q0, tid);
    if (tid < kTile) {
      const bool in = q0 + tid < phi;
      sR[tid] = in ? a.rows[(size_t)head * a.tq_pad + q0 + tid] : make_float2(INFINITY, 0.f);
      if (MASKED) sN[tid] = in ? a.nodes[q0 + tid] : make_int2(-1, -1);
      if (DROP) sKey[tid] = drop_row(a.drop, q0 + tid, head);
    }
    __syncthreads();
    if (!valid) continue;
#pragma unroll
    for (int i = 0; i < kTile; ++i) {
      const int2 pn = MASKED ? sN[i] : make_int2(0, 0);
      if (!admissible_f32<MASKED>(q0 + i, phi, oi, pn, own)) continue;
      const float2 rs = sR[i];
      const float p = fast_exp2(a.c * dotn<HD>(kx, sQ[i]) - rs.x);
      const bool keep = !DROP || drop_keep(a.drop, sKey[i], ck, oc);
      axpyn<HD>(keep ? p : 0.f, sG[i], dv);
      float dp = dotn<HD>(vx, sG[i]);
      if (DROP) dp = keep ? dp * a.drop.inv_keep : 0.f;
      const float ds = p * (dp - rs.y);
      axpyn<HD>(ds, sQ[i], dk);
    }
  }
  if (!valid) return;
  storen<HD>(a.dv + ((size_t)oi * H + head) * HD, dv, DROP ? a.drop.inv_keep : 1.f);
  storen<HD>(a.dk + ((size_t)oi * H + head) * HD, dk, a.scale);
}

// ======================================================================== prep kernel
// One launch whose blocks split into independent tasks.  Per call (fp32
// kernels): a per-segment plan per direction (one block each) and the row
// statistics of the backward pass.  Edge-mask plan build: the packed node
// pairs and per-tile node metadata, the per-token segment bounds of both
// directions, the plan's flag and zero overflow counts.  Blocks are
// dispatched in enum order: the latency-bound tasks (the one-block plans,
// the per-tile metadata, the small per-token tables) come first, so they run
// beside the bandwidth-bound row statistics instead of after them.

enum PrepTask { kPlanQ, kPlanK, kMeta, kNodes, kBoundsQ, kBoundsK, kRows, kPrepTasks };

struct PrepArgs {
  const int* cu_q; const int* cu_k; int nseg;
  int total_q, total_k, heads, tq_pad, tk_pad;
  int head_dim;                        // backward row statistics (fp32): dims per head row
  int4* plan_q; int4* plan_k;          // fp32: per-segment plans (seg_plan_block), plan_k backward only
  int* count_q; int* count_k;          // fp32: their group counts
  int2* bounds_q; int2* bounds_k;      // edge plan
  const bf16* dout; const bf16* out; const float* lse; float c; uint2* aux;   // backward (bf16)
  const float* dout_f; const float* out_f; float2* rows_f;                  // backward (fp32)
  const int* tok_src; const int* tok_dst; int2* nodes; int4* meta;          // masked
  int* over_count;                     // edge plan: the two overflow-list counts, zeroed here
  int* flags; int sym;                 // edge plan: flags[0] = sym (query and key segments coincide)
  int nb[kPrepTasks];                  // blocks per task, in dispatch order
};

// Row statistics of the dK/dV pass, as bf16 (hi, lo) pairs (x = hi + lo to
// ~2^-16 relative): aux.x for -LSE2/c (LSE2 = log2(e) LSE), aux.y for
// -D = -rowsum(dO * O).  Rows without keys and padding get -LSE2/c = -1e30
// (their P is 0).  Thread per (query, head), head fastest.
DEVI void rowstats_item(const PrepArgs& p, long idx) {
  if (idx >= (long)p.heads * p.tq_pad) return;
  const int h = (int)(idx % p.heads), t = (int)(idx / p.heads);
  if (p.rows_f) {
    // fp32 path: (LSE2 = log2(e) LSE, or +inf for rows without keys, D).
    float l2 = INFINITY, d = 0.f;
    if (t < p.total_q) {
      const float l = p.lse[(size_t)h * p.total_q + t];
      if (l != -INFINITY) l2 = l * kLog2e;
      const float4* po = reinterpret_cast<const float4*>(p.out_f + ((size_t)t * p.heads + h) * p.head_dim);
      const float4* pg = reinterpret_cast<const float4*>(p.dout_f + ((size_t)t * p.heads + h) * p.head_dim);
      for (int i = 0; i < p.head_dim / 4; ++i) {
        const float4 o = po[i], g = pg[i];
        d = fmaf(g.x, o.x, d); d = fmaf(g.y, o.y, d); d = fmaf(g.z, o.z, d); d = fmaf(g.w, o.w, d);
      }
    }
    p.rows_f[(size_t)h * p.tq_pad + t] = make_float2(l2, d);
    return;
  }
  float xs = kDeadRow, dsum = 0.f;
  if (t < p.total_q) {
    const float l = p.lse[(size_t)h * p.total_q + t];
    if (l != -INFINITY) xs = -(l * kLog2e) / p.c;
    const bf16x8* po = reinterpret_cast<const bf16x8*>(p.out + ((size_t)t * p.heads + h) * kHd);
    const bf16x8* pd = reinterpret_cast<const bf16x8*>(p.dout + ((size_t)t * p.heads + h) * kHd);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const bf16x8 o = po[j], g = pd[j];
#pragma unroll
      for (int e = 0; e < 8; ++e) dsum = fmaf((float)o[e], (float)g[e], dsum);
    }
  }
  p.aux[(size_t)h * p.tq_pad + t] = make_uint2(split_bf16_pair(xs), split_bf16_pair(-dsum));
}

// Per outer token: the partner range of its segment; padding tokens get an
// empty range.
DEVI void bounds_item(const int* __restrict__ cu_outer, const int* __restrict__ cu_inner, int nseg, int total,
                      int tpad, int2* __restrict__ bounds, int t) {
  if (t >= tpad) return;
  int2 b = make_int2(0, 0);
  if (t < total) {
    const int sg = seg_of(cu_outer, nseg, t);
    b = make_int2(cu_inner[sg], cu_inner[sg + 1]);
  }
  bounds[t] = b;
}

// Per 32-token tile, one wave: min / max node id over both endpoints and a
// 64-bit signature of (node & 63).  Lanes 0-31 read the tile's src ids and
// lanes 32-63 its dst ids (two coalesced loads), then butterfly reductions.
DEVI void meta_wave(const int* __restrict__ src, const int* __restrict__ dst, int total, int4* __restrict__ meta,
                    int tile, int lane) {
  const int t = tile * kTile + (lane & 31);
  const bool in = t < total;
  const int v = in ? (lane < 32 ? src[t] : dst[t]) : 0;
  int lo = in ? v : INT_MAX, hi = in ? v : INT_MIN;
  unsigned sig_lo = in && (v & 63) < 32 ? 1u << (v & 31) : 0u;
  unsigned sig_hi = in && (v & 63) >= 32 ? 1u << (v & 31) : 0u;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    lo = min(lo, __shfl_xor(lo, o));
    hi = max(hi, __shfl_xor(hi, o));
    sig_lo |= __shfl_xor(sig_lo, o);
    sig_hi |= __shfl_xor(sig_hi, o);
  }
  if (lane == 0) meta[tile] = make_int4(lo, hi, (int)sig_lo, (int)sig_hi);
}

__global__ __launch_bounds__(256) void prep_kernel(const PrepArgs p) {
  const int tid = threadIdx.x;
  int b = blockIdx.x;
  if (b < p.nb[kPlanQ]) {
    seg_plan_block(p.cu_q, p.cu_k, p.nseg, kGroupTok, p.plan_q, p.count_q, tid);
    return;
  }
  b -= p.nb[kPlanQ];
  if (b < p.nb[kPlanK]) {
    seg_plan_block(p.cu_k, p.cu_q, p.nseg, kGroupTok, p.plan_k, p.count_k, tid);
    return;
  }
  b -= p.nb[kPlanK];
  if (b < p.nb[kMeta]) {
    const int tile = (b * 256 + tid) >> 6;   // wave-uniform
    if (tile < p.tq_pad / kTile) meta_wave(p.tok_src, p.tok_dst, p.total_q, p.meta, tile, tid & 63);
    return;
  }
  b -= p.nb[kMeta];
  if (b < p.nb[kNodes]) {
    if (b == 0 && tid < 2) p.over_count[tid] = 0;
    if (b == 0 && tid == 0) p.flags[0] = p.sym;
    const int t = b * 256 + tid;
    if (t < p.tq_pad) p.nodes[t] = t < p.total_q ? make_int2(p.tok_src[t], p.tok_dst[t]) : make_int2(-1, -1);
    return;
  }
  b -= p.nb[kNodes];
  if (b < p.nb[kBoundsQ]) { bounds_item(p.cu_q, p.cu_k, p.nseg, p.total_q, p.tq_pad, p.bounds_q, b * 256 + tid); return; }
  b -= p.nb[kBoundsQ];
  if (b < p.nb[kBoundsK]) { bounds_item(p.cu_k, p.cu_q, p.nseg, p.total_k, p.tk_pad, p.bounds_k, b * 256 + tid); return; }
  b -= p.nb[kBoundsK];
  if (b < p.nb[kRows]) rowstats_item(p, (long)b * 256 + tid);
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

// ======================================================================== PMA seed pooling
// k seed queries shared by all B sets (PMA = MAB(S.repeat(B, 1, 1), X)):
// the expanded query row b * k + s is seed s, and set b's queries are rows
// [b k, (b + 1) k).  The seed gradient sums the B sets' rows in set order.
__global__ void pma_expand_kernel(const uint4* __restrict__ q, int row16, int k_seeds, int batch,
                                  uint4* __restrict__ q_rep, int* __restrict__ cu_q) {
  const long n = (long)batch * k_seeds * row16;
  const long i0 = (long)blockIdx.x * blockDim.x + threadIdx.x;
  for (long i = i0; i < n; i += (long)gridDim.x * blockDim.x) {
    const long row = i / row16;
    q_rep[i] = q[(row % k_seeds) * row16 + (i - row * row16)];
  }
  if (i0 <= batch) cu_q[i0] = (int)i0 * k_seeds;
}

template <typename T>
__global__ void pma_reduce_kernel(const T* __restrict__ dq_rep, int row_elems, int k_seeds, int batch,
                                  T* __restrict__ dq) {
  const long n = (long)k_seeds * row_elems;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    float acc = 0.f;
    for (int b = 0; b < batch; ++b) acc += (float)dq_rep[(long)b * n + i];
    dq[i] = (T)acc;
  }
}

// ======================================================================== host side

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
int round32(int x) { return (x + kTile - 1) / kTile * kTile; }
int groups_of(int total) { return (total + kGroupTok - 1) / kGroupTok; }

// ---- edge-mask plans
// The per-batch data of the share-an-endpoint mask, shared by every attention
// call over the same tokens and segments (the reference builds its mask once
// per batch and passes it to every masked layer): the packed node pairs, the
// per-tile node metadata, the per-token partner ranges of both directions,
// the key lists of the query tiles and, when the query and key segments are
// not the same array, of the key tiles, with their overflow groups.  The key
// tiles' lists come last, so their offsets do not depend on whether they
// exist; a flag word tells the dK/dV passes which lists to read.
struct PlanLayout {
  size_t flags = 0, nodes = 0, meta = 0, bounds_q = 0, bounds_k = 0, over_count = 0;
  size_t info[2] = {0, 0}, ids[2] = {0, 0}, bits[2] = {0, 0}, over[2] = {0, 0};
  size_t prep_end = 0;   // end of the sections the prep launch writes (all the fp32 kernels read)
  size_t total = 0;
};

PlanLayout plan_layout(int total_q, int total_k, bool key_lists) {
  PlanLayout P;
  const int tqp = round32(total_q), tkp = round32(total_k);
  size_t off = 0;
  P.flags = off; off += 256;
  P.nodes = off; off += align256((size_t)tqp * 8);
  P.meta = off; off += align256((size_t)(tqp / kTile) * 16);
  P.bounds_q = off; off += align256((size_t)tqp * 8);
  P.bounds_k = off; off += align256((size_t)tkp * 8);
  P.over_count = off; off += 256;
  P.prep_end = off;
  for (int d = 0; d < 2; ++d) {
    const size_t tiles = (size_t)(d ? tkp : tqp) / kTile;
    P.info[d] = off; off += align256(tiles * 4);
    P.ids[d] = off; off += align256(tiles * kListCap * 4);
    P.bits[d] = off; off += align256(tiles * kListCap * 4);
    P.over[d] = off; off += align256((size_t)groups_of(d ? total_k : total_q) * 16);
    if (d == 0) P.total = off;
  }
  if (key_lists) P.total = off;
  return P;
}

// Per-call workspace: the backward row statistics, the fp32 kernels'
// per-segment plans and, for an edge mask given as node ids, the plan the
// call builds (the key tiles' lists only when `key_lists`; for the fp32
// kernels only the prep sections, since they evaluate the predicate from the
// node pairs and read no lists).
struct WsLayout {
  size_t aux = 0, plan_q = 0, plan_k = 0, plan = 0, total = 0;
};

// The edge mask at head dims other than 16, and with attention dropout at
// any head dim, runs the gather kernels over the plan's lists (both dtypes): the plan with its lists, and for the backward
// the per-(head, query) D of the gather kernels, which fits in the aux region.
bool edge_gathered(int mask_kind, int head_dim, bool drop) {
  return (mask_kind == ESA_MASK_EDGE || mask_kind == ESA_MASK_EDGE_PLAN) && (head_dim != kHd || drop);
}

WsLayout ws_layout(int total_q, int total_k, int heads, int dtype, int mask_kind, bool backward, bool key_lists,
                   int head_dim, bool drop) {
  WsLayout L;
  const int tqp = round32(total_q);
  const bool gathered = edge_gathered(mask_kind, head_dim, drop);
  size_t off = 0;
  if (backward) { L.aux = off; off += align256((size_t)heads * tqp * 8); }   // bf16: uint2 (hi, lo); fp32: float2
  if (dtype == ESA_F32 && !gathered) {
    // a 16-byte group count, then per-segment groups (at most ceil(T / 128) + number of segments <= T)
    auto plan_size = [&](int t) { return align256(16 + ((size_t)groups_of(t) + t + 1) * 16); };
    L.plan_q = off; off += plan_size(total_q);
    if (backward) { L.plan_k = off; off += plan_size(total_k); }
  }
  if (mask_kind == ESA_MASK_EDGE) {
    const PlanLayout P = plan_layout(total_q, total_k, key_lists);
    L.plan = off;
    off += dtype == ESA_F32 && !gathered ? align256(P.prep_end) : P.total;
  }
  L.total = off;
  return L;
}

// Device pointers into a built plan.
struct PlanView {
  const int* flags; const int2* nodes; const int4* meta; const int2* bounds_q; const int2* bounds_k;
  const int* over_count; const int* info[2]; const int* ids[2]; const uint32_t* bits[2]; const int4* over[2];
};
PlanView plan_view(const void* plan, int total_q, int total_k) {
  const PlanLayout P = plan_layout(total_q, total_k, true);
  const char* b = static_cast<const char*>(plan);
  PlanView V;
  V.flags = reinterpret_cast<const int*>(b + P.flags);
  V.nodes = reinterpret_cast<const int2*>(b + P.nodes);
  V.meta = reinterpret_cast<const int4*>(b + P.meta);
  V.bounds_q = reinterpret_cast<const int2*>(b + P.bounds_q);
  V.bounds_k = reinterpret_cast<const int2*>(b + P.bounds_k);
  V.over_count = reinterpret_cast<const int*>(b + P.over_count);
  for (int d = 0; d < 2; ++d) {
    V.info[d] = reinterpret_cast<const int*>(b + P.info[d]);
    V.ids[d] = reinterpret_cast<const int*>(b + P.ids[d]);
    V.bits[d] = reinterpret_cast<const uint32_t*>(b + P.bits[d]);
    V.over[d] = reinterpret_cast<const int4*>(b + P.over[d]);
  }
  return V;
}

// ---- edge-mask plan decode (debug): the admissible partners of every outer
// token as the attention kernels read them from a plan.  One wave per outer
// tile, lane l (< 32) for its token l.
//  - A listed tile (info n >= 0): the ceil(n / 32) compact tiles the list
//    kernels visit; bit k of the lane's word c selects list entry 32 c + k
//    (the kernels' score seed), whose id is the partner (a set bit over a -1
//    pad is decoded as -1: the kernels would attend a zero row there).
//  - An overflowing tile (info -1): the walk kernels take its 128-token group
//    only if the group is on the overflow list; they visit the partner tiles
//    of the wave's range that pass the tile-metadata test and keep the
//    partners in the lane's range, other than the token itself, that share an
//    endpoint with it.  A group missing from the list decodes as no partners.
// Direction 1 is what the dK/dV passes read: the key tiles' own lists, or the
// query tiles' when the plan's flag says the mask is symmetric.  Without
// indptr the kernel writes each outer token's partner count to out[t]; with
// indptr (the counts' exclusive scan) the partners, ascending, to
// out[indptr[t] ..].
__global__ __launch_bounds__(256) void edge_plan_decode_kernel(const PlanView V, int dir, int total,
                                                               const int* __restrict__ indptr,
                                                               int* __restrict__ out) {
  const int lane = threadIdx.x & 63, col = lane & 31, half = lane >> 5;
  const int tile = (int)blockIdx.x * kWaves + (threadIdx.x >> 6), o0 = tile * kTile;
  if (o0 >= total) return;   // wave-uniform
  const int ld = (dir == 1 && V.flags[0] != 0) ? 0 : dir;
  const OuterTile ot = outer_tile(dir ? V.bounds_k : V.bounds_q, total, o0, col);
  const bool mine = ot.valid && half == 0;
  const bool fill = indptr != nullptr;
  int* dst = fill && mine ? out + indptr[ot.oi] : nullptr;
  int cnt = 0;
  const int n = V.info[ld][tile];
  if (n >= 0) {
    const int* ids = V.ids[ld] + (size_t)tile * kListCap;
    const uint32_t* bits = V.bits[ld] + (size_t)tile * kListCap;
    for (int c = 0; c * kTile < n; ++c) {
      uint32_t w = mine ? bits[c * kTile + col] : 0u;
      while (w) {
        const int k = __builtin_ctz(w);
        w &= w - 1u;
        if (dst) dst[cnt] = ids[c * kTile + k];
        ++cnt;
      }
    }
  } else {
    const int g = tile / kWaves;
    bool listed = false;
    for (int i = 0; i < V.over_count[ld]; ++i) listed = listed || V.over[ld][i].x == g;
    if (listed) {
      const int4 own = V.meta[tile];
      const int2 qn = V.nodes[ot.oc];
      for (int pt = ot.pt_beg; pt < ot.pt_end; ++pt) {
        if (!tiles_may_touch(own, V.meta[pt])) continue;   // wave-uniform
        for (int j = 0; j < kTile; ++j) {
          const int p = pt * kTile + j;
          if (mine && p >= ot.plo && p < ot.phi && p != ot.oi && node_adjacent(V.nodes[p], qn)) {
            if (dst) dst[cnt] = p;
            ++cnt;
          }
        }
      }
    }
  }
  if (!fill && mine) out[ot.oi] = cnt;
}

bool misaligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; }

// Head dims: 16 on every path; 24, 32 and 64 on the node-mode and edge-mask
// gather kernels, the fp32 kernels and the dense bf16 kernels of
// esa_attn_wide.hip.
bool head_dim_ok(int head_dim) { return head_dim == 16 || head_dim == 24 || head_dim == 32 || head_dim == 64; }

int check_common(int batch, int total_q, int total_k, int heads, int head_dim, int dtype, int mask_kind) {
  if (!head_dim_ok(head_dim)) return ESA_ERR_HEAD_DIM;
  if (dtype != ESA_BF16 && dtype != ESA_F32) return ESA_ERR_DTYPE;
  if (batch < 1 || heads < 1 || total_q < 0 || total_k < 0) return ESA_ERR_SHAPE;
  // Buffer-resource ranges are 32-bit byte counts.
  const long lim = (1L << 31) - 1, row = (long)heads * head_dim * (dtype == ESA_F32 ? 4 : 2);
  if ((long)round32(total_q) * row > lim || (long)round32(total_k) * row > lim) return ESA_ERR_SHAPE;
  if (mask_kind != ESA_MASK_NONE && mask_kind != ESA_MASK_EDGE && mask_kind != ESA_MASK_NODE &&
      mask_kind != ESA_MASK_EDGE_PLAN && mask_kind != ESA_MASK_NODE_PLAN)
    return ESA_ERR_MASK;
  if ((mask_kind == ESA_MASK_EDGE || mask_kind == ESA_MASK_EDGE_PLAN) && total_q != total_k) return ESA_ERR_MASK;
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

int blocks_for(long items) { return (int)((items + 255) / 256); }

enum : unsigned { kTaskPlanQ = 1u, kTaskPlanK = 2u, kTaskMask = 4u, kTaskRows = 8u };

// One prep launch over the selected tasks (kTaskMask: the edge-mask plan's
// node pairs, tile metadata, both directions' bounds, flag and counts).
int launch_prep(PrepArgs& p, unsigned tasks, hipStream_t st) {
  p.nb[kPlanQ] = (tasks & kTaskPlanQ) ? 1 : 0;
  p.nb[kPlanK] = (tasks & kTaskPlanK) ? 1 : 0;
  p.nb[kRows] = (tasks & kTaskRows) ? blocks_for((long)p.heads * p.tq_pad) : 0;
  const bool mask = (tasks & kTaskMask) != 0;
  p.nb[kBoundsQ] = mask ? blocks_for(p.tq_pad) : 0;
  p.nb[kBoundsK] = mask ? blocks_for(p.tk_pad) : 0;
  p.nb[kNodes] = mask ? blocks_for(p.tq_pad) : 0;
  p.nb[kMeta] = mask ? blocks_for((long)(p.tq_pad / kTile) * 64) : 0;
  long grid = 0;
  for (int i = 0; i < kPrepTasks; ++i) grid += p.nb[i];
  if (grid == 0) return ESA_OK;
  ESA_TIMED(esa_profile::kAttnPrep, st,
            hipLaunchKernelGGL(prep_kernel, dim3((unsigned)grid), dim3(256), 0, st, p));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

// Blocks of a one-wave-per-block list kernel: 32-token tiles x head ranges,
// rounded up to whole XCD rounds.
unsigned list_tile_blocks(int total, unsigned n_hw) {
  const unsigned n = (unsigned)((total + kTile - 1) / kTile) * n_hw;
  return (n + kXcds - 1) / kXcds * kXcds;
}

#ifndef ESA_OVERFLOW_GROUPS
#define ESA_OVERFLOW_GROUPS 64
#endif
constexpr int kOverflowGroups = ESA_OVERFLOW_GROUPS;   // groups in flight in a walk kernel over the overflow list
unsigned overflow_blocks(int total) { return (unsigned)std::min(groups_of(total), kOverflowGroups); }

// Builds an edge-mask plan: one prep launch (node pairs, tile metadata,
// bounds, flag, zero counts), then the key lists of the query tiles and, when
// `key_lists`, of the key tiles.  The flag is 1 without key-tile lists (the
// query and key segments are one array: the mask is symmetric).
int build_edge_plan(const int* tok_src, const int* tok_dst, const int* cu_q, const int* cu_k, int batch,
                    int total_q, int total_k, void* plan, bool key_lists, hipStream_t st, bool lists = true) {
  const PlanLayout P = plan_layout(total_q, total_k, key_lists);
  char* b = static_cast<char*>(plan);
  PrepArgs pa{};
  pa.cu_q = cu_q; pa.cu_k = cu_k; pa.nseg = batch;
  pa.total_q = total_q; pa.total_k = total_k; pa.heads = 1;
  pa.tq_pad = round32(total_q); pa.tk_pad = round32(total_k);
  pa.tok_src = tok_src; pa.tok_dst = tok_dst;
  pa.nodes = reinterpret_cast<int2*>(b + P.nodes);
  pa.meta = reinterpret_cast<int4*>(b + P.meta);
  pa.bounds_q = reinterpret_cast<int2*>(b + P.bounds_q);
  pa.bounds_k = reinterpret_cast<int2*>(b + P.bounds_k);
  pa.over_count = reinterpret_cast<int*>(b + P.over_count);
  pa.flags = reinterpret_cast<int*>(b + P.flags);
  pa.sym = key_lists ? 0 : 1;
  int rc = launch_prep(pa, kTaskMask, st);
  if (rc || !lists) return rc;
  ListArgs la{};
  la.nodes = pa.nodes; la.meta = pa.meta;
  la.total = total_q;
  la.n_groups = groups_of(total_q);
  la.bounds[0] = pa.bounds_q; la.bounds[1] = pa.bounds_k;
  for (int d = 0; d < 2; ++d) {
    la.info[d] = reinterpret_cast<int*>(b + P.info[d]);
    la.ids[d] = reinterpret_cast<int*>(b + P.ids[d]);
    la.bits[d] = reinterpret_cast<uint32_t*>(b + P.bits[d]);
    la.over[d] = reinterpret_cast<int4*>(b + P.over[d]);
    la.over_count[d] = pa.over_count + d;
  }
  const unsigned grid = (unsigned)la.n_groups * (key_lists ? 2u : 1u);
  ESA_TIMED(esa_profile::kAttnEdgeLists, st, hipLaunchKernelGGL(edge_lists_kernel, dim3(grid), dim3(256), 0, st, la));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

// The plan of a masked call: the caller's (ESA_MASK_EDGE_PLAN: mask_a points
// at it) or one built into the call's workspace from the node ids (without
// key lists for the fp32 kernels, which read only the node pairs).
int call_plan(int mask_kind, const int* mask_a, const int* mask_b, const int* cu_q, const int* cu_k, int batch,
              int total_q, int total_k, char* ws, const WsLayout& L, bool key_lists, bool lists, hipStream_t st,
              const void** plan) {
  if (mask_kind == ESA_MASK_EDGE_PLAN) {
    *plan = mask_a;
    return ESA_OK;
  }
  *plan = ws + L.plan;
  return build_edge_plan(mask_a, mask_b, cu_q, cu_k, batch, total_q, total_k, ws + L.plan, key_lists, st, lists);
}

// Arguments of the gather kernels for the edge mask at head dims 32 / 64: the
// plan's lists, node pairs, flag and per-token partner ranges.
GraphAttnArgs edge_gather_args(const void* plan, const void* q, const void* k, const void* v, const int* cu_q,
                               const int* cu_k, int batch, int total_q, int total_k, int heads, int head_dim,
                               float scale) {
  const PlanView V = plan_view(plan, total_q, total_k);
  GraphAttnArgs g{};
  g.q = q; g.k = k; g.v = v; g.cu_q = cu_q; g.cu_k = cu_k; g.nseg = batch;
  g.total_q = total_q; g.total_k = total_k; g.heads = heads; g.head_dim = head_dim;
  g.c = scale * kLog2e; g.scale = scale;
  g.q_bounds = V.bounds_q; g.k_bounds = V.bounds_k;
  g.edge.sym = V.flags; g.edge.nodes = V.nodes; g.edge.cap = kListCap;
  for (int d = 0; d < 2; ++d) {
    g.edge.info[d] = V.info[d];
    g.edge.ids[d] = V.ids[d];
    g.edge.bits[d] = V.bits[d];
  }
  return g;
}

// KERNEL<false, HD, DROP> (the fp32 kernels without a mask) for head dim 16, 24, 32 or 64.
#define ESA_F32_LAUNCH_HD(KERNEL, D, hd, grid, st, a)                                                \
  do {                                                                                               \
    if (hd == 16) hipLaunchKernelGGL((KERNEL<false, 16, D>), grid, dim3(kF32Threads), 0, st, a);      \
    else if (hd == 24) hipLaunchKernelGGL((KERNEL<false, 24, D>), grid, dim3(kF32Threads), 0, st, a); \
    else if (hd == 32) hipLaunchKernelGGL((KERNEL<false, 32, D>), grid, dim3(kF32Threads), 0, st, a); \
    else hipLaunchKernelGGL((KERNEL<false, 64, D>), grid, dim3(kF32Threads), 0, st, a);              \
  } while (0)
constexpr unsigned kF32FwdThreads(int hd) { return kF32Threads * (hd >= 64 ? f32_splits<64>() : f32_splits<16>()); }
#define ESA_F32_FWD_HD(D, hd, grid, st, a)                                                                 \
  do {                                                                                                     \
    if (hd == 16)                                                                                          \
      hipLaunchKernelGGL((attn_fwd_f32_kernel<false, 16, D>), grid, dim3(kF32FwdThreads(16)), 0, st, a);    \
    else if (hd == 24)                                                                                     \
      hipLaunchKernelGGL((attn_fwd_f32_kernel<false, 24, D>), grid, dim3(kF32FwdThreads(24)), 0, st, a);    \
    else if (hd == 32)                                                                                     \
      hipLaunchKernelGGL((attn_fwd_f32_kernel<false, 32, D>), grid, dim3(kF32FwdThreads(32)), 0, st, a);    \
    else                                                                                                   \
      hipLaunchKernelGGL((attn_fwd_f32_kernel<false, 64, D>), grid, dim3(kF32FwdThreads(64)), 0, st, a);    \
  } while (0)
// Unmasked fp32 calls whose max_seqlen_q is 1..kFewQueries take the few-query kernels (the forward at
// every head dim, the backward at head dims up to kFewBwdMaxHd: a dK/dV thread holds six rows of the head dim).
constexpr int kFewQueries = 4, kFewBwdMaxHd = 32;
template <bool D>
void few_launch(int which, int hd, dim3 grid, hipStream_t st, const AttnFewArgs& a) {
#define ESA_FEW_K(KERNEL, HD) hipLaunchKernelGGL((KERNEL<HD, D>), grid, dim3(256), 0, st, a)
#define ESA_FEW_HD(KERNEL)                                       \
  do {                                                           \
    if (hd == 16) ESA_FEW_K(KERNEL, 16);                         \
    else if (hd == 24) ESA_FEW_K(KERNEL, 24);                    \
    else ESA_FEW_K(KERNEL, 32);                                  \
  } while (0)
  if (which == 0) {
    if (hd == 64) ESA_FEW_K(attn_fwd_few_kernel, 64);
    else ESA_FEW_HD(attn_fwd_few_kernel);
  } else if (which == 1) {
    ESA_FEW_HD(attn_dq_few_kernel);
  } else {
    ESA_FEW_HD(attn_dkdv_few_kernel);
  }
#undef ESA_FEW_HD
#undef ESA_FEW_K
}
void few_go(int which, bool drop, int hd, dim3 grid, hipStream_t st, const AttnFewArgs& a) {
  if (drop) few_launch<true>(which, hd, grid, st, a); else few_launch<false>(which, hd, grid, st, a);
}
// Arguments of the few-query kernels; the forward and dQ grid (waves per segment: slots x heads, 4 per block).
AttnFewArgs few_args(const void* q, const void* k, const void* v, const int* cu_q, const int* cu_k, int nseg,
                     int total_q, int total_k, int heads, int slots, float scale, const DropoutCfg& drop) {
  AttnFewArgs f{};
  f.q = static_cast<const float*>(q); f.k = static_cast<const float*>(k); f.v = static_cast<const float*>(v); f.cu_q = cu_q; f.cu_k = cu_k; f.nseg = nseg;
  f.total_q = total_q; f.total_k = total_k; f.heads = heads; f.slots = slots;
  f.blocks_per_seg = (slots * heads + 3) / 4;
  f.c = scale * kLog2e; f.scale = scale; f.drop = drop;
  return f;
}

#define ESA_F32_FWD_LAUNCH(hd, drop, grid, st, a)  \
  do {                                             \
    if (drop) ESA_F32_FWD_HD(true, hd, grid, st, a); \
    else ESA_F32_FWD_HD(false, hd, grid, st, a);     \
  } while (0)
#define ESA_F32_LAUNCH(KERNEL, hd, drop, grid, st, a)                                                \
  do {                                                                                               \
    if (drop) ESA_F32_LAUNCH_HD(KERNEL, true, hd, grid, st, a);                                     \
    else ESA_F32_LAUNCH_HD(KERNEL, false, hd, grid, st, a);                                         \
  } while (0)

// Scratch of esa_varlen_attn_fwd_noalloc: a file-scope device array, one
// copy per GPU, held until the process ends.  Host code never passes the
// array's name (a host-side stand-in) to a kernel: it passes the device
// address hipGetSymbolAddress returns, looked up once per device on the
// first call with that device current.
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return ESA_ERR_SHAPE;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!ptr) return ESA_ERR_NULL;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return ESA_OK;
}

}  // namespace

extern "C" {

const char* esa_version(void) { return "esa_hip 0.3 gfx950"; }

int esa_varlen_attn_workspace_size(int total_q, int total_k, int heads, int head_dim, int dtype, int mask_kind,
                                   int n_mask_edges, int backward, size_t* bytes) {
  if (!bytes) return ESA_ERR_NULL;
  const int rc = check_common(1, total_q, total_k, heads, head_dim, dtype, mask_kind);
  if (rc) return rc;
  if (mask_kind == ESA_MASK_NODE || mask_kind == ESA_MASK_NODE_PLAN) {
    if (n_mask_edges < 0) return ESA_ERR_SHAPE;
    return graph_attn_workspace_size(total_q, total_k, heads, n_mask_edges, backward != 0,
                                     mask_kind == ESA_MASK_NODE_PLAN, bytes);
  }
  if (mask_kind == ESA_MASK_NONE && dtype == ESA_BF16)
    return dense_attn_workspace_size(total_q, total_k, heads, head_dim, backward != 0, bytes);
  // a backward call that builds its plan may need the key tiles' lists (distinct segment arrays); the
  // size covers the calls with and without dropout (which may take different kernels)
  *bytes = std::max(ws_layout(total_q, total_k, heads, dtype, mask_kind, backward != 0, backward != 0, head_dim,
                              false).total,
                    ws_layout(total_q, total_k, heads, dtype, mask_kind, backward != 0, backward != 0, head_dim,
                              true).total);
  return ESA_OK;
}

int esa_edge_plan_size(int total_q, int total_k, int symmetric, size_t* bytes) {
  if (!bytes) return ESA_ERR_NULL;
  if (total_q < 0 || total_k < 0 || total_q != total_k) return ESA_ERR_SHAPE;
  *bytes = plan_layout(total_q, total_k, symmetric == 0).total;
  return ESA_OK;
}

int esa_edge_plan_build(const int* tok_src, const int* tok_dst, const int* cu_seqlens_q, const int* cu_seqlens_k,
                        int batch, int total_q, int total_k, void* plan, size_t plan_bytes, void* stream) {
  if (!tok_src || !tok_dst || !cu_seqlens_q || !cu_seqlens_k || !plan) return ESA_ERR_NULL;
  if (batch < 1 || total_q < 0 || total_q != total_k) return ESA_ERR_SHAPE;
  if (misaligned(plan)) return ESA_ERR_ALIGN;
  const bool key_lists = cu_seqlens_q != cu_seqlens_k;
  if (plan_bytes < plan_layout(total_q, total_k, key_lists).total) return ESA_ERR_WORKSPACE;
  if (total_q == 0) return ESA_OK;
  return build_edge_plan(tok_src, tok_dst, cu_seqlens_q, cu_seqlens_k, batch, total_q, total_k, plan, key_lists,
                         reinterpret_cast<hipStream_t>(stream));
}

int esa_node_plan_size(int total_q, int total_k, int n_mask_edges, size_t* bytes) {
  if (!bytes) return ESA_ERR_NULL;
  if (total_q < 0 || total_k < 0 || n_mask_edges < 0) return ESA_ERR_SHAPE;
  return graph_node_plan_size(total_q, total_k, n_mask_edges, bytes);
}

int esa_node_plan_build(const int* indptr, const int* indices, const int* cu_seqlens_q, const int* cu_seqlens_k,
                        int batch, int total_q, int total_k, int n_mask_edges, void* plan, size_t plan_bytes,
                        void* stream) {
  if (!indptr || !plan || !cu_seqlens_q || !cu_seqlens_k || (n_mask_edges > 0 && !indices)) return ESA_ERR_NULL;
  if (batch < 1 || total_q < 0 || total_k < 0 || n_mask_edges < 0) return ESA_ERR_SHAPE;
  if (misaligned(plan)) return ESA_ERR_ALIGN;
  return graph_node_plan_build(indptr, indices, cu_seqlens_q, cu_seqlens_k, batch, total_q, total_k, n_mask_edges,
                               plan, plan_bytes, reinterpret_cast<hipStream_t>(stream));
}

int esa_varlen_attn_fwd(const void* q, const void* k, const void* v, const int* cu_seqlens_q,
                        const int* cu_seqlens_k, int batch, int total_q, int total_k,
                        int max_seqlen_q, int max_seqlen_k, int heads, int head_dim, int dtype,
                        float softmax_scale, float dropout_p, unsigned long long dropout_seed, int mask_kind,
                        const int* mask_a, const int* mask_b, int n_mask_edges, void* out, float* softmax_lse,
                        void* workspace, size_t workspace_bytes, void* stream) {
  (void)max_seqlen_k;   // max_seqlen_q routes fp32 calls with few queries per segment; results never depend on it
  int rc = check_common(batch, total_q, total_k, heads, head_dim, dtype, mask_kind);
  if (rc) return rc;
  if (!(dropout_p >= 0.f && dropout_p < 1.f)) return ESA_ERR_DROPOUT;
  const bool drop = dropout_p > 0.f;
  const DropoutCfg dcfg = make_dropout(dropout_p, dropout_seed, heads);
  if (mask_kind == ESA_MASK_NODE || mask_kind == ESA_MASK_NODE_PLAN) {
    if (n_mask_edges < 0) return ESA_ERR_SHAPE;
    if (!mask_a || ((n_mask_edges > 0 || mask_kind == ESA_MASK_NODE_PLAN) && !mask_b)) return ESA_ERR_NULL;
    if (mask_kind == ESA_MASK_NODE_PLAN && misaligned(mask_b)) return ESA_ERR_ALIGN;
    if (total_q == 0) return ESA_OK;
    if (!q || !k || !v || !cu_seqlens_q || !cu_seqlens_k || !out || !softmax_lse) return ESA_ERR_NULL;
    if (misaligned(q) || misaligned(k) || misaligned(v) || misaligned(out)) return ESA_ERR_ALIGN;
    if (!(softmax_scale > 0.f)) return ESA_ERR_SHAPE;
    GraphAttnArgs g{};
    g.q = q; g.k = k; g.v = v; g.cu_q = cu_seqlens_q; g.cu_k = cu_seqlens_k; g.nseg = batch;
    g.total_q = total_q; g.total_k = total_k; g.heads = heads; g.head_dim = head_dim;
    g.indptr = mask_a; g.indices = mask_b; g.nnz = n_mask_edges;
    g.c = softmax_scale * kLog2e; g.scale = softmax_scale;
    g.drop = dcfg; g.dropout = drop;
    g.out = out; g.lse = softmax_lse;
    (void)workspace; (void)workspace_bytes;
    return graph_attn_fwd(g, dtype, mask_kind == ESA_MASK_NODE_PLAN ? mask_b : nullptr,
                          reinterpret_cast<hipStream_t>(stream));
  }
  const bool masked = mask_kind == ESA_MASK_EDGE || mask_kind == ESA_MASK_EDGE_PLAN;
  if (mask_kind == ESA_MASK_EDGE && (!mask_a || !mask_b)) return ESA_ERR_NULL;
  if (mask_kind == ESA_MASK_EDGE_PLAN && !mask_a) return ESA_ERR_NULL;
  if (total_q == 0) return ESA_OK;
  if (!q || !k || !v || !cu_seqlens_q || !cu_seqlens_k || !out || !softmax_lse) return ESA_ERR_NULL;
  if (misaligned(q) || misaligned(k) || misaligned(v) || misaligned(out) || misaligned(workspace)) return ESA_ERR_ALIGN;
  if (!(softmax_scale > 0.f)) return ESA_ERR_SHAPE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool f32 = dtype == ESA_F32;
  if (f32 && !masked && max_seqlen_q > 0 && max_seqlen_q <= kFewQueries) {   // the PMA's seeds: no workspace
    AttnFewArgs fa = few_args(q, k, v, cu_seqlens_q, cu_seqlens_k, batch, total_q, total_k, heads, max_seqlen_q,
                              softmax_scale, dcfg);
    fa.o = static_cast<float*>(out); fa.lse_out = softmax_lse;
    ESA_TIMED(esa_profile::kAttnFwd, st,
              few_go(0, drop, head_dim, dim3((unsigned)batch * (unsigned)fa.blocks_per_seg), st, fa));
    ESA_LAUNCH_CHECK();
    return ESA_OK;
  }
  if (!masked && !f32) {
    if (!workspace) return ESA_ERR_NULL;
    DenseAttnCall c{};
    c.q = q; c.k = k; c.v = v; c.cu_q = cu_seqlens_q; c.cu_k = cu_seqlens_k; c.nseg = batch;
    c.total_q = total_q; c.total_k = total_k; c.heads = heads; c.head_dim = head_dim; c.scale = softmax_scale;
    c.drop = dcfg; c.dropout = drop;
    c.out = out; c.lse = softmax_lse;
    return dense_attn_fwd(c, workspace, workspace_bytes, st);
  }
  const bool gathered = edge_gathered(mask_kind, head_dim, drop);
  const WsLayout L = ws_layout(total_q, total_k, heads, dtype, mask_kind, false, false, head_dim, drop);
  if (workspace_bytes < L.total) return ESA_ERR_WORKSPACE;
  if (L.total && !workspace) return ESA_ERR_NULL;
  char* ws = static_cast<char*>(workspace);
  const void* plan = nullptr;
  if (masked && (rc = call_plan(mask_kind, mask_a, mask_b, cu_seqlens_q, cu_seqlens_k, batch, total_q, total_k, ws,
                                L, false, !f32 || gathered, st, &plan)))
    return rc;

  if (gathered) {   // the edge mask at head dims 24 / 32 / 64 or with dropout: gather kernels over the plan's lists
    GraphAttnArgs g = edge_gather_args(plan, q, k, v, cu_seqlens_q, cu_seqlens_k, batch, total_q, total_k, heads,
                                       head_dim, softmax_scale);
    g.drop = dcfg; g.dropout = drop;
    g.out = out; g.lse = softmax_lse;
    return graph_edge_attn_fwd(g, dtype, st);
  }
  if (f32) {
    PrepArgs pa{};
    pa.cu_q = cu_seqlens_q; pa.cu_k = cu_seqlens_k; pa.nseg = batch;
    pa.total_q = total_q; pa.total_k = total_k; pa.heads = heads;
    pa.tq_pad = round32(total_q); pa.tk_pad = round32(total_k);
    pa.plan_q = reinterpret_cast<int4*>(ws + L.plan_q + 16);
    pa.count_q = reinterpret_cast<int*>(ws + L.plan_q);
    if ((rc = launch_prep(pa, kTaskPlanQ, st))) return rc;
    AttnF32Args a{};
    a.q = static_cast<const float*>(q); a.k = static_cast<const float*>(k); a.v = static_cast<const float*>(v);
    a.total_q = total_q; a.total_k = total_k; a.heads = heads; a.tq_pad = pa.tq_pad;
    a.c = softmax_scale * kLog2e; a.scale = softmax_scale;
    a.drop = dcfg;
    a.nodes = masked ? plan_view(plan, total_q, total_k).nodes : nullptr;
    a.plan = pa.plan_q; a.count = pa.count_q;
    a.o = static_cast<float*>(out); a.lse_out = softmax_lse;
    const dim3 fgrid((unsigned)(groups_of(total_q) + batch) * (unsigned)heads);
    if (masked)   // head_dim 16 without dropout (the rest take the gather kernels)
      ESA_TIMED(esa_profile::kAttnFwdMasked, st,
                hipLaunchKernelGGL((attn_fwd_f32_kernel<true, 16, false>), fgrid, dim3(kF32FwdThreads(16)), 0, st, a));
    else
      ESA_TIMED(esa_profile::kAttnFwd, st, ESA_F32_FWD_LAUNCH(head_dim, drop, fgrid, st, a));
    ESA_LAUNCH_CHECK();
    return ESA_OK;
  }

  // bf16 edge mask: the key-list forward, then the walk kernel over the overflowing groups
  const PlanView V = plan_view(plan, total_q, total_k);
  AttnArgs a{};
  a.q = static_cast<const bf16*>(q); a.k = static_cast<const bf16*>(k); a.v = static_cast<const bf16*>(v);
  a.cu_q = cu_seqlens_q; a.cu_k = cu_seqlens_k; a.nseg = batch;
  a.total_q = total_q; a.total_k = total_k; a.heads = heads; a.tq_pad = round32(total_q);
  a.tk_tiles = round32(total_k) / kTile;
  a.scale = softmax_scale; a.c = softmax_scale * kLog2e;
  a.bounds = V.bounds_q;
  a.nodes = V.nodes; a.meta = V.meta;
  a.info = V.info[0]; a.ids = V.ids[0]; a.bits = V.bits[0];
  a.o = static_cast<bf16*>(out); a.lse_out = softmax_lse;
  const unsigned n_hq = ((heads + kListHeads - 1) / kListHeads + kWaves - 1) / kWaves;
  ESA_TIMED(esa_profile::kAttnFwdMasked, st,
            hipLaunchKernelGGL(list_fwd_kernel, dim3(list_tile_blocks(total_q, n_hq)), dim3(256), 0, st, a));
  ESA_LAUNCH_CHECK();
  a.plan = V.over[0];
  a.count = V.over_count;
  const unsigned n_hg_walk = (unsigned)((heads + kEdgeHeads - 1) / kEdgeHeads);
  ESA_TIMED(esa_profile::kAttnEdgeOverflow, st,
            hipLaunchKernelGGL(edge_fwd_kernel, dim3(overflow_blocks(total_q) * n_hg_walk), dim3(256), 0, st, a));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

size_t esa_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int esa_varlen_attn_fwd_noalloc(const void* q, const void* k, const void* v, const int* cu_seqlens_q,
                                const int* cu_seqlens_k, int batch, int total_q, int total_k,
                                int max_seqlen_q, int max_seqlen_k, int heads, int head_dim, int dtype,
                                float softmax_scale, float dropout_p, unsigned long long dropout_seed,
                                int mask_kind, const int* mask_a, const int* mask_b, int n_mask_edges, void* out,
                                float* softmax_lse, void* stream) {
  size_t need = 0;
  int rc = esa_varlen_attn_workspace_size(total_q, total_k, heads, head_dim, dtype, mask_kind, n_mask_edges, 0,
                                          &need);
  if (rc) return rc;
  if (need > kNoAllocScratchBytes) return ESA_ERR_SCRATCH;
  void* ws = nullptr;
  if ((rc = scratch_address(&ws))) return rc;
  // The prep pass writes every scratch word the forward kernels read, as it
  // does for the allocating entry point's uninitialised workspace, so nothing
  // needs clearing between calls.
  return esa_varlen_attn_fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, batch, total_q, total_k, max_seqlen_q,
                             max_seqlen_k, heads, head_dim, dtype, softmax_scale, dropout_p, dropout_seed, mask_kind,
                             mask_a, mask_b, n_mask_edges, out, softmax_lse, ws, kNoAllocScratchBytes, stream);
}

int esa_varlen_attn_bwd(const void* dout, const void* q, const void* k, const void* v, const void* out,
                        const float* softmax_lse, const int* cu_seqlens_q, const int* cu_seqlens_k,
                        int batch, int total_q, int total_k, int max_seqlen_q, int max_seqlen_k,
                        int heads, int head_dim, int dtype, float softmax_scale, float dropout_p,
                        unsigned long long dropout_seed, int mask_kind, const int* mask_a, const int* mask_b,
                        int n_mask_edges, void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes,
                        void* stream) {
  (void)max_seqlen_k;   // max_seqlen_q routes calls with few queries per segment; results never depend on it
  int rc = check_common(batch, total_q, total_k, heads, head_dim, dtype, mask_kind);
  if (rc) return rc;
  if (!(dropout_p >= 0.f && dropout_p < 1.f)) return ESA_ERR_DROPOUT;
  const bool drop = dropout_p > 0.f;
  const DropoutCfg dcfg = make_dropout(dropout_p, dropout_seed, heads);
  if (mask_kind == ESA_MASK_NODE || mask_kind == ESA_MASK_NODE_PLAN) {
    const bool planned = mask_kind == ESA_MASK_NODE_PLAN;
    if (n_mask_edges < 0) return ESA_ERR_SHAPE;
    if (!mask_a || ((n_mask_edges > 0 || planned) && !mask_b)) return ESA_ERR_NULL;
    if (planned && misaligned(mask_b)) return ESA_ERR_ALIGN;
    if (total_q == 0 && total_k == 0) return ESA_OK;
    if (!dout || !q || !k || !v || !out || !softmax_lse || !cu_seqlens_q || !cu_seqlens_k || !dq || !dk || !dv ||
        !workspace)
      return ESA_ERR_NULL;
    if (misaligned(dout) || misaligned(q) || misaligned(k) || misaligned(v) || misaligned(out) || misaligned(dq) ||
        misaligned(dk) || misaligned(dv) || misaligned(workspace))
      return ESA_ERR_ALIGN;
    if (!(softmax_scale > 0.f)) return ESA_ERR_SHAPE;
    GraphAttnArgs g{};
    g.q = q; g.k = k; g.v = v; g.cu_q = cu_seqlens_q; g.cu_k = cu_seqlens_k; g.nseg = batch;
    g.total_q = total_q; g.total_k = total_k; g.heads = heads; g.head_dim = head_dim;
    g.indptr = mask_a; g.indices = mask_b; g.nnz = n_mask_edges;
    g.c = softmax_scale * kLog2e; g.scale = softmax_scale;
    g.drop = dcfg; g.dropout = drop;
    g.out_in = out; g.dout = dout; g.lse_in = softmax_lse;
    g.dq = dq; g.dk = dk; g.dv = dv;
    return graph_attn_bwd(g, dtype, planned ? mask_b : nullptr, workspace, workspace_bytes,
                          reinterpret_cast<hipStream_t>(stream));
  }
  const bool masked = mask_kind == ESA_MASK_EDGE || mask_kind == ESA_MASK_EDGE_PLAN;
  if (mask_kind == ESA_MASK_EDGE && (!mask_a || !mask_b)) return ESA_ERR_NULL;
  if (mask_kind == ESA_MASK_EDGE_PLAN && !mask_a) return ESA_ERR_NULL;
  if (total_q == 0 && total_k == 0) return ESA_OK;
  if (!dout || !q || !k || !v || !out || !softmax_lse || !cu_seqlens_q || !cu_seqlens_k || !dq || !dk ||
      !dv || !workspace)
    return ESA_ERR_NULL;
  if (misaligned(dout) || misaligned(q) || misaligned(k) || misaligned(v) || misaligned(out) ||
      misaligned(dq) || misaligned(dk) || misaligned(dv) || misaligned(workspace))
    return ESA_ERR_ALIGN;
  if (!(softmax_scale > 0.f)) return ESA_ERR_SHAPE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool f32 = dtype == ESA_F32;
  const size_t esz = f32 ? 4 : 2;
  if (total_q == 0 || total_k == 0) {
    // No query/key pairs: every gradient is zero (a fill kernel, so the call
    // stays capturable in a HIP graph).
    if ((rc = launch_zero(dq, (size_t)total_q * heads * head_dim * esz, st))) return rc;
    if ((rc = launch_zero(dk, (size_t)total_k * heads * head_dim * esz, st))) return rc;
    if ((rc = launch_zero(dv, (size_t)total_k * heads * head_dim * esz, st))) return rc;
    return ESA_OK;
  }
  if (f32 && !masked && max_seqlen_q > 0 && max_seqlen_q <= kFewQueries && head_dim <= kFewBwdMaxHd) {
    // the PMA's seeds: dQ (writing the row statistics at the workspace's start), then dK/dV
    if (workspace_bytes < (size_t)heads * total_q * sizeof(float2)) return ESA_ERR_WORKSPACE;
    AttnFewArgs fa = few_args(q, k, v, cu_seqlens_q, cu_seqlens_k, batch, total_q, total_k, heads, max_seqlen_q,
                              softmax_scale, dcfg);
    fa.out = static_cast<const float*>(out); fa.dout = static_cast<const float*>(dout); fa.lse = softmax_lse;
    fa.rows = static_cast<float2*>(workspace);
    fa.dq = static_cast<float*>(dq); fa.dk = static_cast<float*>(dk); fa.dv = static_cast<float*>(dv);
    ESA_TIMED(esa_profile::kAttnBwdDq, st,
              few_go(1, drop, head_dim, dim3((unsigned)batch * (unsigned)fa.blocks_per_seg), st, fa));
    ESA_TIMED(esa_profile::kAttnBwdDkdv, st,
              few_go(2, drop, head_dim, dim3((unsigned)(((long)total_k * heads + 255) / 256)), st, fa));
    ESA_LAUNCH_CHECK();
    return ESA_OK;
  }
  if (!masked && !f32) {
    DenseAttnCall c{};
    c.q = q; c.k = k; c.v = v; c.cu_q = cu_seqlens_q; c.cu_k = cu_seqlens_k; c.nseg = batch;
    c.total_q = total_q; c.total_k = total_k; c.heads = heads; c.head_dim = head_dim; c.scale = softmax_scale;
    c.out_in = out; c.dout = dout; c.lse_in = softmax_lse; c.dq = dq; c.dk = dk; c.dv = dv;
    c.drop = dcfg; c.dropout = drop;
    return dense_attn_bwd(c, workspace, workspace_bytes, st);
  }
  // A plan built here has the key tiles' own lists when the segment arrays are distinct.
  const bool key_lists = cu_seqlens_q != cu_seqlens_k;
  const bool gathered = edge_gathered(mask_kind, head_dim, drop);
  const WsLayout L = ws_layout(total_q, total_k, heads, dtype, mask_kind, true, key_lists, head_dim, drop);
  if (workspace_bytes < L.total) return ESA_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  const void* plan = nullptr;
  if (masked && (rc = call_plan(mask_kind, mask_a, mask_b, cu_seqlens_q, cu_seqlens_k, batch, total_q, total_k, ws,
                                L, key_lists, !f32 || gathered, st, &plan)))
    return rc;

  if (gathered) {   // the edge mask at head dims 24 / 32 / 64 or with dropout: gather kernels over the plan's lists
    GraphAttnArgs g = edge_gather_args(plan, q, k, v, cu_seqlens_q, cu_seqlens_k, batch, total_q, total_k, heads,
                                       head_dim, softmax_scale);
    g.drop = dcfg; g.dropout = drop;
    g.out_in = out; g.dout = dout; g.lse_in = softmax_lse;
    g.dq = dq; g.dk = dk; g.dv = dv;
    return graph_edge_attn_bwd(g, dtype, ws + L.aux, workspace_bytes - L.aux, st);
  }
  if (f32) {
    PrepArgs pa{};
    pa.cu_q = cu_seqlens_q; pa.cu_k = cu_seqlens_k; pa.nseg = batch;
    pa.total_q = total_q; pa.total_k = total_k; pa.heads = heads;
    pa.tq_pad = round32(total_q); pa.tk_pad = round32(total_k);
    pa.plan_q = reinterpret_cast<int4*>(ws + L.plan_q + 16);
    pa.plan_k = reinterpret_cast<int4*>(ws + L.plan_k + 16);
    pa.count_q = reinterpret_cast<int*>(ws + L.plan_q);
    pa.count_k = reinterpret_cast<int*>(ws + L.plan_k);
    pa.lse = softmax_lse; pa.c = softmax_scale * kLog2e;
    pa.dout_f = static_cast<const float*>(dout); pa.out_f = static_cast<const float*>(out);
    pa.rows_f = reinterpret_cast<float2*>(ws + L.aux);
    pa.head_dim = head_dim;
    if ((rc = launch_prep(pa, kTaskPlanQ | kTaskPlanK | kTaskRows, st))) return rc;
    AttnF32Args a{};
    a.q = static_cast<const float*>(q); a.k = static_cast<const float*>(k); a.v = static_cast<const float*>(v);
    a.out = static_cast<const float*>(out); a.dout = static_cast<const float*>(dout);
    a.rows = pa.rows_f;
    a.total_q = total_q; a.total_k = total_k; a.heads = heads; a.tq_pad = pa.tq_pad;
    a.c = softmax_scale * kLog2e; a.scale = softmax_scale;
    a.drop = dcfg;
    a.nodes = masked ? plan_view(plan, total_q, total_k).nodes : nullptr;
    a.dq = static_cast<float*>(dq); a.dk = static_cast<float*>(dk); a.dv = static_cast<float*>(dv);
    a.plan = pa.plan_k; a.count = pa.count_k;
    const dim3 fkgrid((unsigned)(groups_of(total_k) + batch) * (unsigned)heads);
    const dim3 fqgrid((unsigned)(groups_of(total_q) + batch) * (unsigned)heads);
    if (masked)   // head_dim 16 without dropout (the rest take the gather kernels)
      ESA_TIMED(esa_profile::kAttnBwdDkdvMasked, st,
                hipLaunchKernelGGL((attn_dkdv_f32_kernel<true, 16, false>), fkgrid, dim3(kF32Threads), 0, st, a));
    else
      ESA_TIMED(esa_profile::kAttnBwdDkdv, st, ESA_F32_LAUNCH(attn_dkdv_f32_kernel, head_dim, drop, fkgrid, st, a));
    ESA_LAUNCH_CHECK();
    a.plan = pa.plan_q; a.count = pa.count_q;
    if (masked)
      ESA_TIMED(esa_profile::kAttnBwdDqMasked, st,
                hipLaunchKernelGGL((attn_dq_f32_kernel<true, 16, false>), fqgrid, dim3(kF32Threads), 0, st, a));
    else
      ESA_TIMED(esa_profile::kAttnBwdDq, st, ESA_F32_LAUNCH(attn_dq_f32_kernel, head_dim, drop, fqgrid, st, a));
    ESA_LAUNCH_CHECK();
    return ESA_OK;
  }

  // bf16 edge mask: the dQ list pass first (it writes the row statistics the
  // dK/dV passes read), then the dK/dV list pass, then one launch of the dQ
  // and dK/dV walk kernels over the overflowing groups.
  const PlanView V = plan_view(plan, total_q, total_k);
  AttnArgs a{};
  a.q = static_cast<const bf16*>(q); a.k = static_cast<const bf16*>(k); a.v = static_cast<const bf16*>(v);
  a.out = static_cast<const bf16*>(out); a.dout = static_cast<const bf16*>(dout); a.lse = softmax_lse;
  a.aux = reinterpret_cast<const uint2*>(ws + L.aux);
  a.aux_out = reinterpret_cast<uint2*>(ws + L.aux);
  a.cu_q = cu_seqlens_q; a.cu_k = cu_seqlens_k; a.nseg = batch;
  a.total_q = total_q; a.total_k = total_k; a.heads = heads; a.tq_pad = round32(total_q);
  a.tk_tiles = round32(total_k) / kTile;
  a.scale = softmax_scale; a.c = softmax_scale * kLog2e;
  a.nodes = V.nodes; a.meta = V.meta;
  a.sym = V.flags;
  a.kinfo = V.info[1]; a.kids = V.ids[1]; a.kbits = V.bits[1]; a.kover = V.over[1]; a.kcount = V.over_count + 1;
  a.dq = static_cast<bf16*>(dq); a.dk = static_cast<bf16*>(dk); a.dv = static_cast<bf16*>(dv);

  const unsigned n_hg = (unsigned)((heads + kListHeads - 1) / kListHeads);
  const unsigned n_hg_walk = (unsigned)((heads + kEdgeHeads - 1) / kEdgeHeads);
  a.bounds = V.bounds_q;
  a.info = V.info[0]; a.ids = V.ids[0]; a.bits = V.bits[0];
  ESA_TIMED(esa_profile::kAttnBwdDqMasked, st,
            hipLaunchKernelGGL(list_dq_kernel, dim3(list_tile_blocks(total_q, (n_hg + kWaves - 1) / kWaves)), dim3(256),
                               0, st, a));
  ESA_LAUNCH_CHECK();
  a.plan = V.over[0];
  a.count = V.over_count;
  AttnArgs adq = a;   // the dQ walk's arguments (query tiles' overflow groups and bounds)

  const unsigned n_hg_kv = (unsigned)((heads + kListHeadsKv - 1) / kListHeadsKv);
  const unsigned n_hg_kv_walk = (unsigned)((heads + kEdgeHeadsKv - 1) / kEdgeHeadsKv);
  a.bounds = V.bounds_k;
  ESA_TIMED(esa_profile::kAttnBwdDkdvMasked, st,
            hipLaunchKernelGGL(list_dkdv_kernel, dim3(list_tile_blocks(total_k, (n_hg_kv + kWaves - 1) / kWaves)),
                               dim3(256), 0, st, a));
  ESA_LAUNCH_CHECK();
  const unsigned dq_blocks = overflow_blocks(total_q) * n_hg_walk;
  ESA_TIMED(esa_profile::kAttnEdgeOverflow, st,
            hipLaunchKernelGGL(edge_bwd_walk_kernel, dim3(dq_blocks + overflow_blocks(total_k) * n_hg_kv_walk),
                               dim3(256), 0, st, adq, a, (int)dq_blocks));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

// ---- PMA entry points: expansion + varlen attention (+ seed-gradient reduction)
static int pma_layout(int batch, int k_seeds, int total_k, int heads, int head_dim, int dtype, bool backward,
                      size_t off[4], size_t* total) {
  if (batch < 1 || k_seeds < 1 || total_k < 0 || heads < 1) return ESA_ERR_SHAPE;
  if (!head_dim_ok(head_dim)) return ESA_ERR_HEAD_DIM;
  if (dtype != ESA_BF16 && dtype != ESA_F32) return ESA_ERR_DTYPE;
  const long tq = (long)batch * k_seeds;
  if (tq > INT32_MAX / 2) return ESA_ERR_SHAPE;
  const size_t rows = (size_t)tq * heads * head_dim * (dtype == ESA_F32 ? 4 : 2);
  size_t inner = 0;
  const int rc = esa_varlen_attn_workspace_size((int)tq, total_k, heads, head_dim, dtype, ESA_MASK_NONE, 0,
                                                backward ? 1 : 0, &inner);
  if (rc) return rc;
  size_t o = 0;
  off[0] = o; o += align256(rows);                               // expanded seed queries
  off[1] = o; o += align256((size_t)(batch + 1) * 4);            // cu_seqlens of the expanded queries
  off[2] = o; o += backward ? align256(rows) : 0;                // per-set seed gradients
  off[3] = o; o += inner;                                        // the varlen call's own workspace
  *total = o;
  return ESA_OK;
}

static int pma_expand(const void* q, int batch, int k_seeds, int heads, int head_dim, int dtype, char* ws,
                      const size_t off[4], hipStream_t st) {
  const int row16 = heads * head_dim * (dtype == ESA_F32 ? 4 : 2) / 16;
  const long n = (long)batch * k_seeds * row16;
  const long g = std::min<long>(std::max<long>((n + 255) / 256, (batch + 1 + 255) / 256), 65536);
  hipLaunchKernelGGL(pma_expand_kernel, dim3((unsigned)g), dim3(256), 0, st, static_cast<const uint4*>(q), row16,
                     k_seeds, batch, reinterpret_cast<uint4*>(ws + off[0]), reinterpret_cast<int*>(ws + off[1]));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

int esa_pma_workspace_size(int batch, int k_seeds, int total_k, int heads, int head_dim, int dtype, int backward,
                           size_t* bytes) {
  if (!bytes) return ESA_ERR_NULL;
  size_t off[4];
  return pma_layout(batch, k_seeds, total_k, heads, head_dim, dtype, backward != 0, off, bytes);
}

int esa_pma_fwd(const void* q, const void* k, const void* v, const int* cu_seqlens_k, int batch, int k_seeds,
                int total_k, int max_seqlen_k, int heads, int head_dim, int dtype, float softmax_scale,
                float dropout_p, unsigned long long dropout_seed, void* out, float* softmax_lse, void* workspace,
                size_t workspace_bytes, void* stream) {
  size_t off[4], need = 0;
  int rc = pma_layout(batch, k_seeds, total_k, heads, head_dim, dtype, false, off, &need);
  if (rc) return rc;
  if (!q || !k || !v || !cu_seqlens_k || !out || !softmax_lse || !workspace) return ESA_ERR_NULL;
  if (workspace_bytes < need) return ESA_ERR_WORKSPACE;
  if (misaligned(q) || misaligned(workspace)) return ESA_ERR_ALIGN;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  if ((rc = pma_expand(q, batch, k_seeds, heads, head_dim, dtype, ws, off, st))) return rc;
  return esa_varlen_attn_fwd(ws + off[0], k, v, reinterpret_cast<const int*>(ws + off[1]), cu_seqlens_k, batch,
                             batch * k_seeds, total_k, k_seeds, max_seqlen_k, heads, head_dim, dtype, softmax_scale,
                             dropout_p, dropout_seed, ESA_MASK_NONE, nullptr, nullptr, 0, out, softmax_lse, ws + off[3],
                             need - off[3], stream);
}

int esa_pma_bwd(const void* dout, const void* q, const void* k, const void* v, const void* out,
                const float* softmax_lse, const int* cu_seqlens_k, int batch, int k_seeds, int total_k,
                int max_seqlen_k, int heads, int head_dim, int dtype, float softmax_scale, float dropout_p,
                unsigned long long dropout_seed, void* dq, void* dk, void* dv, void* workspace,
                size_t workspace_bytes, void* stream) {
  size_t off[4], need = 0;
  int rc = pma_layout(batch, k_seeds, total_k, heads, head_dim, dtype, true, off, &need);
  if (rc) return rc;
  if (!dout || !q || !k || !v || !out || !softmax_lse || !cu_seqlens_k || !dq || !dk || !dv || !workspace)
    return ESA_ERR_NULL;
  if (workspace_bytes < need) return ESA_ERR_WORKSPACE;
  if (misaligned(q) || misaligned(workspace)) return ESA_ERR_ALIGN;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  if ((rc = pma_expand(q, batch, k_seeds, heads, head_dim, dtype, ws, off, st))) return rc;
  rc = esa_varlen_attn_bwd(dout, ws + off[0], k, v, out, softmax_lse, reinterpret_cast<const int*>(ws + off[1]),
                           cu_seqlens_k, batch, batch * k_seeds, total_k, k_seeds, max_seqlen_k, heads, head_dim,
                           dtype, softmax_scale, dropout_p, dropout_seed, ESA_MASK_NONE, nullptr, nullptr, 0,
                           ws + off[2], dk, dv, ws + off[3], need - off[3], stream);
  if (rc) return rc;
  const int row_elems = heads * head_dim;
  const long n = (long)k_seeds * row_elems;
  const unsigned g = (unsigned)std::min<long>((n + 255) / 256, 65536);
  if (dtype == ESA_F32)
    hipLaunchKernelGGL(pma_reduce_kernel<float>, dim3(g), dim3(256), 0, st,
                       reinterpret_cast<const float*>(ws + off[2]), row_elems, k_seeds, batch, static_cast<float*>(dq));
  else
    hipLaunchKernelGGL(pma_reduce_kernel<bf16>, dim3(g), dim3(256), 0, st,
                       reinterpret_cast<const bf16*>(ws + off[2]), row_elems, k_seeds, batch, static_cast<bf16*>(dq));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

int esa_edge_plan_decode(const void* plan, int total_q, int total_k, int direction, const int* indptr, int* out,
                         void* stream) {
  if (!plan || !out) return ESA_ERR_NULL;
  if (total_q < 0 || total_q != total_k || (direction != 0 && direction != 1)) return ESA_ERR_SHAPE;
  if (misaligned(plan)) return ESA_ERR_ALIGN;
  if (total_q == 0) return ESA_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned tiles = (unsigned)round32(total_q) / kTile;
  hipLaunchKernelGGL(edge_plan_decode_kernel, dim3((tiles + kWaves - 1) / kWaves), dim3(256), 0, st,
                     plan_view(plan, total_q, total_k), direction, total_q, indptr, out);
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

int esa_node_plan_sections(int total_q, int total_k, int n_mask_edges, size_t* offsets) {
  if (!offsets) return ESA_ERR_NULL;
  if (total_q < 0 || total_k < 0 || n_mask_edges < 0) return ESA_ERR_SHAPE;
  return graph_node_plan_sections(total_q, total_k, n_mask_edges, offsets);
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
