// Gathered (per-token) masked attention on gfx950: node mode, and the edge
// mask at head dims other than 16.
//
// Node mode: query token i attends to the key tokens listed in row i of a CSR
// (indptr [total_q + 1], indices [nnz]): the mask that
// get_adj_mask_from_edge_index_node (esa/masked_layers.py:79-118) builds as a
// padded [B, 1, N, N] bias, 0 at (graph, src_local, dst_local) of every edge
// and -99999 elsewhere, applied by memory_efficient_attention (esa/mha.py:76).
// Rows must list their keys in ascending order; an entry equal to its
// predecessor is a repeated edge and counts once, as repeated writes of 0 into
// the reference's bias do.  Entries outside the query's segment are ignored.
//
// Edge mask (share an endpoint, esa/masked_layers.py:121-142, 217-268) at
// head dims 32 and 64: the same kernels take a token's partners from the
// edge-mask plan, i.e. from its 32-token tile's partner list (the entries
// whose mask bit the token has set, ascending) or, for a tile past the list
// capacity, from the predicate over the token's segment.
//
// The work is O(partners * heads * head_dim) -- a few to a few tens of
// partners per token -- so it is gathered per token instead of tiled for
// MFMA: one wave per token, a power-of-two group of lanes per head with N = 4
// or 8 dims on each lane (N = 4: head dim 16 on 4 lanes, 32 on 8, 64 on 16,
// 24 on 8 lanes of which the last two hold zeros; N = 8 halves the lanes per
// head, so a wave covers 512 dims at once), scores reduced over a head's lanes
// by DPP butterflies (identical in all of them), fp32 online softmax.  Every
// pass of a wave over its heads walks the token's whole partner list, a chain
// of dependent loads, so the launch takes N = 8 where it needs fewer passes
// (dim 512: one pass instead of two).
// The forward and dQ gather over the token's partners; dK / dV over the
// queries that attend to the key (node mode: the transposed CSR, built per
// call with the library's stable CSR sort or once per batch into a node plan;
// edge mask: the key tiles' lists, or the query tiles' when the mask is
// symmetric).  Every sum runs in a fixed order: the backward is deterministic.
// With attention dropout (DROP), each partner's probability enters the
// products over partners only where the call's keep mask (esa_common.h) keeps
// it, and the outputs carry the 1 / (1 - p) factor; the softmax statistics
// are those of the undropped scores.
#include "esa_common.h"
#include "esa_csr.h"
#include "esa_graph_attn.h"
#include "esa_profile.h"
#include "../../include/esa_hip.h"

namespace {

// Partners per step: their K / V (or Q / dO) rows are loaded together; the
// partner indices come from registers (CsrSrc), so a step's row loads wait on
// no index load.  At 4 dims per lane (16 heads of 16, bf16): four for the
// forward and dQ (two: 1-2 % slower, three: 10 % slower), two for dK / dV
// (four: 6 % slower); fp32 rows take two (four would cost the forward and dQ
// their eighth wave per SIMD).  At 8 dims per lane (dim 512): two everywhere
// (one: forward 9 %, dQ 2 %, dK / dV 3 % slower).  Build-time overrides for
// measurement.
#ifndef ESA_NODE_G4
#define ESA_NODE_G4 4
#endif
#ifndef ESA_NODE_G4K
#define ESA_NODE_G4K 2
#endif
#ifndef ESA_NODE_G8
#define ESA_NODE_G8 2
#endif
#ifndef ESA_NODE_G8K
#define ESA_NODE_G8K 2
#endif
template <typename T, int N, bool KEY_SIDE> constexpr int partners_per_step() {
  return N == 8 ? (KEY_SIDE ? ESA_NODE_G8K : ESA_NODE_G8)
                : (KEY_SIDE || sizeof(T) != 2 ? ESA_NODE_G4K : ESA_NODE_G4);
}

template <typename T> struct Row4;
template <> struct Row4<float> { typedef f32x4 type; };
template <> struct Row4<bf16> { typedef bf16x4 type; };

// N (4 or 8) consecutive values of a [T][H][head_dim] row: this lane's dims
// of one head, as 16-byte (or, fp32 at N = 4, one 16-byte; bf16 at N = 4, one
// 8-byte) loads and stores.
template <typename T, int N>
DEVI void load_dims(const T* __restrict__ p, float v[N]) {
#pragma unroll
  for (int c = 0; c < N / 4; ++c) {
    const typename Row4<T>::type x = reinterpret_cast<const typename Row4<T>::type*>(p)[c];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[4 * c + i] = (float)x[i];
  }
}
template <typename T, int N>
DEVI void store_dims(T* __restrict__ p, const float v[N], float mul) {
#pragma unroll
  for (int c = 0; c < N / 4; ++c) {
    typename Row4<T>::type x;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = (T)(v[4 * c + i] * mul);
    reinterpret_cast<typename Row4<T>::type*>(p)[c] = x;
  }
}

template <int CTRL>
DEVI float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// Sum over the L lanes of a head (aligned groups of 2, 4, 8 or 16 lanes):
// butterflies within each quad ([1,0,3,2], [2,3,0,1]), then the other quad of
// each half row (row_half_mirror) and the other half of each row (row_mirror).  Addition is commutative, so every lane of the group
// holds the identical result.
template <int L>
DEVI float head_sum(float x) {
  x += dpp<0xB1>(x);
  if (L >= 4) x += dpp<0x4E>(x);
  if (L >= 8) x += dpp<0x141>(x);
  if (L >= 16) x += dpp<0x140>(x);
  return x;
}
template <int N>
DEVI float dotn(const float a[N], const float b[N]) {
  float s = a[0] * b[0];
#pragma unroll
  for (int i = 1; i < N; ++i) s = fmaf(a[i], b[i], s);
  return s;
}

// Lanes of one head: HD / N of them carry N dims each, rounded up to a power
// of two (head dim 24, N = 4: 6 of 8).  A lane past the head's dims reads the
// last dims (an in-row address), zeroes its own token's operand so that its
// terms of every dot product are 0, and stores nothing.
template <int HD, int N>
struct HeadLanes {
  static_assert(N == 4 || (N == 8 && HD % 16 == 0), "8 dims per lane need a head dim of 16, 32 or 64");
  static constexpr int L = HD == 24 ? 8 : HD / N;
  static constexpr int HPP = 64 / L;   // heads per pass of a wave
  int li, d0;
  bool dims;
  DEVI HeadLanes(int lane) : li(lane % L), d0(N * min(lane % L, HD / N - 1)), dims(lane % L < HD / N) {}
  DEVI void own(float v[N]) const {
    if (HD / N == L) return;
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = dims ? v[i] : 0.f;
  }
};

// fp32 path: the device library's exp2f / log2f; bf16 path: the hardware
// approximations (as in the tiled kernels).
template <typename T> DEVI float ex2(float x) { return fast_exp2(x); }
template <> DEVI float ex2<float>(float x) { return exp2f(x); }
template <typename T> DEVI float lg2(float x) { return fast_log2(x); }
template <> DEVI float lg2<float>(float x) { return log2f(x); }

// Segment of the wave's token t (wave-uniform): the largest s in [0, nseg)
// with cu[s] <= t, as seg_of's binary search finds it, but with the wave's
// 64 lanes sampling the range at once: each round narrows it 64-fold with one
// load per lane and a ballot (two rounds up to 4096 segments, instead of
// log2(nseg) dependent loads).
DEVI int wave_seg_of(const int* __restrict__ cu, int nseg, int t) {
  const int lane = threadIdx.x & 63;
  int base = 0, span = nseg;
  while (span > 1) {
    const int step = (span + 63) >> 6, end = base + span;
    const int s = base + lane * step;
    const uint64_t m = __ballot(s < end && cu[s] <= t);
    if (m == 0) break;   // cu[base] > t: only possible at base 0 (seg_of's answer as well)
    base += (63 - __builtin_clzll(m)) * step;
    span = min(step, end - base);
  }
  return base;
}

// Row [pa, pb) of a CSR clamped into [0, nnz).
DEVI void csr_row(const int* __restrict__ indptr, int t, int nnz, int& pa, int& pb) {
  pa = min(max(indptr[t], 0), nnz);
  pb = min(max(indptr[t + 1], pa), nnz);
}

// Token descriptor {lo, hi, pa, pb}: the partner range [lo, hi) of token t
// (segment sg by cu_own, range by cu_other) and its CSR row [pa, pb), emptied
// when the range is.  A node plan stores them: one 16-byte load per token
// instead of the segment search, the range and the row bounds (forward, dQ
// and dK / dV 7-11 % faster); without a plan they are computed here.
DEVI int4 make_desc(const int* __restrict__ cu_other, int total_other, const int* __restrict__ indptr, int nnz,
                    int sg, int t) {
  const int lo = max(cu_other[sg], 0), hi = min(cu_other[sg + 1], total_other);
  int pa, pb;
  csr_row(indptr, t, nnz, pa, pb);
  return make_int4(lo, hi, pa, hi > lo ? pb : pa);
}
DEVI int4 token_desc(const int4* __restrict__ plan_desc, const int* __restrict__ cu_own,
                     const int* __restrict__ cu_other, int nseg, int total_other, const int* __restrict__ indptr,
                     int nnz, int t) {
  if (plan_desc) return plan_desc[t];
  return make_desc(cu_other, total_other, indptr, nnz, wave_seg_of(cu_own, nseg, t), t);
}

// This wave's token (one wave per token, four waves per block; more tokens per
// wave, each wave walking a run of them with the next token's descriptor in
// flight, measured slower: a fresh wave per token keeps every slot busy).
// Hardware block b runs on XCD b % 8; blocks are dealt so that each XCD takes
// one contiguous range of tokens, whose partners (mostly nearby tokens of the
// same graph) are then read into that XCD's L2.
DEVI int wave_token() {
  const int nb = gridDim.x, q = nb >> 3, rem = nb & 7, x = blockIdx.x & 7, s = blockIdx.x >> 3;
  const int b = x * q + min(x, rem) + s;
  return b * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// ---- partner sources: next<G>(j, ok) yields the next G partners of the
// wave's token (j a valid row index even where !ok), false once exhausted.  The
// walk position and the partners yielded are wave-uniform (a source may hold a
// block of entries spread over the lanes); a copy restarts the walk (one per
// head pass).

// A CSR row [p, pb): entries in [lo, hi), each once (an entry equal to its
// predecessor is a repeat).  The row is read 64 entries at a time by one
// vector load (lane l holds entry base + l) and a step takes its entries by
// readlane, so the partner rows of a step wait on no index load of their own.
struct CsrSrc {
  const int* list; int p, pb, lo, hi, prev, base, blk;
  DEVI void fill() {
    const int i = base + (int)(threadIdx.x & 63);
    blk = i < pb ? list[i] : 0;
  }
  template <int G>
  DEVI bool next(int (&j)[G], bool (&ok)[G]) {
    if (p >= pb) return false;
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const int pp = p + u;
      int x = prev;
      if (pp < pb) {
        if (pp >= base + 64) {   // wave-uniform: the next 64 entries
          base += 64;
          fill();
        }
        x = __builtin_amdgcn_readlane(blk, pp - base);
      }
      ok[u] = pp < pb && x >= lo && x < hi && x != prev;
      if (pp < pb) prev = x;
      j[u] = ok[u] ? x : lo;
    }
    p += G;
    return true;
  }
};

// An edge-mask plan's list for one token: the entries of its tile's list
// whose mask bit the token has set, in list (= ascending token) order.  Word
// c of the token's mask bits is held by lane c (at most kListCap / 32 words);
// the 32 ids of word c's entries are held by lanes 0..31 (one vector load per
// word) and taken by readlane, so no partner waits on an id load of its own.
struct ListSrc {
  const int* ids; uint32_t words; int nct, c; uint32_t w; int fallback, idv;
  DEVI void fetch() { idv = ids[32 * c + (int)(threadIdx.x & 31)]; }
  template <int G>
  DEVI bool next(int (&j)[G], bool (&ok)[G]) {
    bool any = false;
#pragma unroll
    for (int u = 0; u < G; ++u) {
      if (w == 0u && c + 1 < nct) {   // wave-uniform: the next word with a set bit
        do {
          ++c;
          w = (uint32_t)__builtin_amdgcn_readlane((int)words, c);
        } while (w == 0u && c + 1 < nct);
        fetch();
      }
      ok[u] = w != 0u;
      j[u] = fallback;
      if (ok[u]) {
        j[u] = __builtin_amdgcn_readlane(idv, __builtin_ctz(w));
        w &= w - 1u;
        any = true;
      }
    }
    return any;
  }
};
DEVI ListSrc list_src(const GraphEdgeLists& e, int d, int t, int n) {
  const int lane = threadIdx.x & 63, tile = t >> 5;
  ListSrc s;
  s.ids = e.ids[d] + (size_t)tile * e.cap;
  s.nct = (n + 31) >> 5;
  s.words = lane < s.nct ? e.bits[d][(size_t)tile * e.cap + 32 * lane + (t & 31)] : 0u;
  s.c = 0;
  s.w = s.nct > 0 ? (uint32_t)__builtin_amdgcn_readlane((int)s.words, 0) : 0u;
  s.fallback = t;
  s.idv = 0;
  if (s.nct > 0) s.fetch();
  return s;
}

// A token of a tile past the list capacity: the partners p in [lo, hi), p !=
// t, that share an endpoint with t, 64 candidates per ballot.
struct WalkSrc {
  const int2* nodes; int2 own; int t, base, hi, cur; uint64_t mask;
  template <int G>
  DEVI bool next(int (&j)[G], bool (&ok)[G]) {
    const int lane = threadIdx.x & 63;
    bool any = false;
#pragma unroll
    for (int u = 0; u < G; ++u) {
      while (mask == 0 && base < hi) {
        const int p = base + lane;
        bool keep = false;
        if (p < hi && p != t) {
          const int2 n = nodes[p];
          keep = n.x == own.x || n.x == own.y || n.y == own.x || n.y == own.y;
        }
        mask = __ballot(keep);
        cur = base;
        base += 64;
      }
      ok[u] = mask != 0;
      j[u] = t;
      if (ok[u]) {
        j[u] = cur + __builtin_ctzll(mask);
        mask &= mask - 1;
        any = true;
      }
    }
    return any;
  }
};
DEVI WalkSrc walk_src(const GraphEdgeLists& e, int2 bounds, int t) {
  WalkSrc s;
  s.nodes = e.nodes;
  s.own = e.nodes[t];
  s.t = t;
  s.base = bounds.x;
  s.hi = bounds.y;
  s.cur = 0;
  s.mask = 0;
  return s;
}

template <typename T, int HD, int N, bool DROP, class Src>
DEVI void fwd_token(const GraphAttnArgs& a, int t, const Src& src0) {
  constexpr int L = HeadLanes<HD, N>::L, HPP = HeadLanes<HD, N>::HPP, G = partners_per_step<T, N, false>();
  const T* __restrict__ q = static_cast<const T*>(a.q);
  const T* __restrict__ k = static_cast<const T*>(a.k);
  const T* __restrict__ v = static_cast<const T*>(a.v);
  const int lane = threadIdx.x & 63, H = a.heads;
  const HeadLanes<HD, N> hl(lane);
  const int d0 = hl.d0;
  for (int h0 = 0; h0 < H; h0 += HPP) {
    const int h = h0 + lane / L;
    const int hc = min(h, H - 1);
    float qv[N], acc[N];
#pragma unroll
    for (int i = 0; i < N; ++i) acc[i] = 0.f;
    load_dims<T, N>(q + ((size_t)t * H + hc) * HD + d0, qv);
    hl.own(qv);
    const uint32_t rk = DROP ? drop_row(a.drop, t, hc) : 0u;
    float m = -INFINITY, l = 0.f;
    Src src = src0;
    int j[G];
    bool ok[G];
    while (src.template next<G>(j, ok)) {
      float kr[G][N], vr[G][N];
#pragma unroll
      for (int u = 0; u < G; ++u) {
        load_dims<T, N>(k + ((size_t)j[u] * H + hc) * HD + d0, kr[u]);
        load_dims<T, N>(v + ((size_t)j[u] * H + hc) * HD + d0, vr[u]);
      }
      float s[G];
      float mt = m;
#pragma unroll
      for (int u = 0; u < G; ++u) {
        s[u] = ok[u] ? head_sum<L>(dotn<N>(qv, kr[u])) * a.c : -INFINITY;
        mt = fmaxf(mt, s[u]);
      }
      if (mt == -INFINITY) continue;   // nothing admissible yet (uniform per head)
      const float alpha = ex2<T>(m - mt);   // 0 while m = -inf
      l *= alpha;
#pragma unroll
      for (int i = 0; i < N; ++i) acc[i] *= alpha;
#pragma unroll
      for (int u = 0; u < G; ++u) {
        const float pu = ex2<T>(s[u] - mt);
        l += pu;
        const float pv = !DROP || drop_keep(a.drop, rk, drop_col(a.drop, j[u]), j[u]) ? pu : 0.f;
#pragma unroll
        for (int i = 0; i < N; ++i) acc[i] = fmaf(pv, vr[u][i], acc[i]);
      }
      m = mt;
    }
    if (h < H) {
      if (hl.dims)
        store_dims<T, N>(static_cast<T*>(a.out) + ((size_t)t * H + h) * HD + d0, acc,
                  l > 0.f ? (DROP ? a.drop.inv_keep : 1.f) / l : 0.f);
      if (hl.li == 0) a.lse[(size_t)h * a.total_q + t] = l > 0.f ? (m + lg2<T>(l)) * kLn2 : -INFINITY;
    }
  }
}

// dQ_i = scale * sum_j P_ij (dP_ij - D_i) k_j over i's partners; also writes
// D_i = rowsum(dO_i * O_i) per head for the dK / dV pass.
template <typename T, int HD, int N, bool DROP, class Src>
DEVI void dq_token(const GraphAttnArgs& a, int t, const Src& src0) {
  constexpr int L = HeadLanes<HD, N>::L, HPP = HeadLanes<HD, N>::HPP, G = partners_per_step<T, N, false>();
  const T* __restrict__ q = static_cast<const T*>(a.q);
  const T* __restrict__ k = static_cast<const T*>(a.k);
  const T* __restrict__ v = static_cast<const T*>(a.v);
  const T* __restrict__ o = static_cast<const T*>(a.out_in);
  const T* __restrict__ g = static_cast<const T*>(a.dout);
  const int lane = threadIdx.x & 63, H = a.heads;
  const HeadLanes<HD, N> hl(lane);
  const int d0 = hl.d0;
  for (int h0 = 0; h0 < H; h0 += HPP) {
    const int h = h0 + lane / L;
    const int hc = min(h, H - 1);
    const size_t row = ((size_t)t * H + hc) * HD + d0;
    float qv[N], gv[N], ov[N], acc[N];
#pragma unroll
    for (int i = 0; i < N; ++i) acc[i] = 0.f;
    load_dims<T, N>(q + row, qv);
    load_dims<T, N>(g + row, gv);
    load_dims<T, N>(o + row, ov);
    hl.own(qv);
    hl.own(gv);
    const float dsum = head_sum<L>(dotn<N>(gv, ov));
    const uint32_t rk = DROP ? drop_row(a.drop, t, hc) : 0u;
    const float l = a.lse_in[(size_t)hc * a.total_q + t];
    const float l2 = l == -INFINITY ? INFINITY : l * kLog2e;
    if (h < H && hl.li == 0) a.dsum[(size_t)h * a.total_q + t] = dsum;
    Src src = src0;
    int j[G];
    bool ok[G];
    while (src.template next<G>(j, ok)) {
      float kr[G][N], vr[G][N];
#pragma unroll
      for (int u = 0; u < G; ++u) {
        load_dims<T, N>(k + ((size_t)j[u] * H + hc) * HD + d0, kr[u]);
        load_dims<T, N>(v + ((size_t)j[u] * H + hc) * HD + d0, vr[u]);
      }
#pragma unroll
      for (int u = 0; u < G; ++u) {
        const float pu = ok[u] ? ex2<T>(fmaf(head_sum<L>(dotn<N>(qv, kr[u])), a.c, -l2)) : 0.f;
        float dp = head_sum<L>(dotn<N>(gv, vr[u]));
        if (DROP) dp = drop_keep(a.drop, rk, drop_col(a.drop, j[u]), j[u]) ? dp * a.drop.inv_keep : 0.f;
        const float ds = pu * (dp - dsum);
#pragma unroll
        for (int i = 0; i < N; ++i) acc[i] = fmaf(ds, kr[u][i], acc[i]);
      }
    }
    if (h < H && hl.dims) store_dims<T, N>(static_cast<T*>(a.dq) + ((size_t)t * H + h) * HD + d0, acc, a.scale);
  }
}

// dV_j = sum_i P_ij dO_i, dK_j = scale * sum_i P_ij (dP_ij - D_i) q_i over the
// queries i that attend to key j (ascending).
template <typename T, int HD, int N, bool DROP, class Src>
DEVI void dkdv_token(const GraphAttnArgs& a, int t, const Src& src0) {
  constexpr int L = HeadLanes<HD, N>::L, HPP = HeadLanes<HD, N>::HPP, G = partners_per_step<T, N, true>();
  const T* __restrict__ q = static_cast<const T*>(a.q);
  const T* __restrict__ k = static_cast<const T*>(a.k);
  const T* __restrict__ v = static_cast<const T*>(a.v);
  const T* __restrict__ g = static_cast<const T*>(a.dout);
  const int lane = threadIdx.x & 63, H = a.heads;
  const HeadLanes<HD, N> hl(lane);
  const int d0 = hl.d0;
  for (int h0 = 0; h0 < H; h0 += HPP) {
    const int h = h0 + lane / L;
    const int hc = min(h, H - 1);
    const size_t row = ((size_t)t * H + hc) * HD + d0;
    float kv[N], vv[N], dk[N], dv[N];
#pragma unroll
    for (int i = 0; i < N; ++i) dk[i] = dv[i] = 0.f;
    load_dims<T, N>(k + row, kv);
    load_dims<T, N>(v + row, vv);
    hl.own(kv);
    hl.own(vv);
    const uint32_t ck = DROP ? drop_col(a.drop, t) : 0u;
    Src src = src0;
    int i[G];
    bool ok[G];
    while (src.template next<G>(i, ok)) {
      float qr[G][N], gr[G][N], l2[G], ds_[G];
#pragma unroll
      for (int u = 0; u < G; ++u) {
        const size_t r = ((size_t)i[u] * H + hc) * HD + d0;
        load_dims<T, N>(q + r, qr[u]);
        load_dims<T, N>(g + r, gr[u]);
        l2[u] = a.lse_in[(size_t)hc * a.total_q + i[u]] * kLog2e;
        ds_[u] = a.dsum[(size_t)hc * a.total_q + i[u]];
      }
#pragma unroll
      for (int u = 0; u < G; ++u) {
        const float pu = ok[u] ? ex2<T>(fmaf(head_sum<L>(dotn<N>(qr[u], kv)), a.c, -l2[u])) : 0.f;
        float dp = head_sum<L>(dotn<N>(gr[u], vv)), pv = pu;
        if (DROP && !drop_keep(a.drop, drop_row(a.drop, i[u], hc), ck, t)) dp = pv = 0.f;
        if (DROP) dp *= a.drop.inv_keep;
        const float ds = pu * (dp - ds_[u]);
#pragma unroll
        for (int c = 0; c < N; ++c) {
          dv[c] = fmaf(pv, gr[u][c], dv[c]);
          dk[c] = fmaf(ds, qr[u][c], dk[c]);
        }
      }
    }
    if (h < H && hl.dims) {
      store_dims<T, N>(static_cast<T*>(a.dk) + ((size_t)t * H + h) * HD + d0, dk, a.scale);
      store_dims<T, N>(static_cast<T*>(a.dv) + ((size_t)t * H + h) * HD + d0, dv, DROP ? a.drop.inv_keep : 1.f);
    }
  }
}

DEVI CsrSrc csr_src(const int* list, int4 d) {
  CsrSrc s{list, d.z, d.w, d.x, d.y, INT_MIN, d.z, 0};
  s.fill();
  return s;
}

// The kernels: node mode over a CSR (the key pass over the transposed CSR).
template <typename T, int HD, int N, bool DROP>
__global__ __launch_bounds__(256) void graph_attn_fwd_kernel(const GraphAttnArgs a) {
  const int t = wave_token();
  if (t >= a.total_q) return;
  fwd_token<T, HD, N, DROP>(a, t, csr_src(a.indices, token_desc(a.q_desc, a.cu_q, a.cu_k, a.nseg, a.total_k, a.indptr, a.nnz, t)));
}
template <typename T, int HD, int N, bool DROP>
__global__ __launch_bounds__(256) void graph_attn_dq_kernel(const GraphAttnArgs a) {
  const int t = wave_token();
  if (t >= a.total_q) return;
  dq_token<T, HD, N, DROP>(a, t, csr_src(a.indices, token_desc(a.q_desc, a.cu_q, a.cu_k, a.nseg, a.total_k, a.indptr, a.nnz, t)));
}
template <typename T, int HD, int N, bool DROP>
__global__ __launch_bounds__(256) void graph_attn_dkdv_kernel(const GraphAttnArgs a) {
  const int t = wave_token();
  if (t >= a.total_k) return;
  dkdv_token<T, HD, N, DROP>(a, t, csr_src(a.t_rows, token_desc(a.k_desc, a.cu_k, a.cu_q, a.nseg, a.total_q, a.t_indptr, a.nnz, t)));
}

// Edge mask over a plan's lists: the query side reads direction 0, the key
// side direction 1, or direction 0 when the plan is symmetric.
template <typename T, int HD, int N, bool DROP, int PASS>   // 0 forward, 1 dQ, 2 dK / dV
DEVI void graph_edge_pass(const GraphAttnArgs& a) {
  const int t = wave_token();
  if (t >= (PASS == 2 ? a.total_k : a.total_q)) return;
  const int d = (PASS == 2 && a.edge.sym[0] == 0) ? 1 : 0;
  const int n = a.edge.info[d][t >> 5];
  auto run = [&](const auto& src) {
    if (PASS == 0) fwd_token<T, HD, N, DROP>(a, t, src);
    if (PASS == 1) dq_token<T, HD, N, DROP>(a, t, src);
    if (PASS == 2) dkdv_token<T, HD, N, DROP>(a, t, src);
  };
  if (n >= 0)
    run(list_src(a.edge, d, t, n));
  else
    run(walk_src(a.edge, (PASS == 2 ? a.k_bounds : a.q_bounds)[t], t));
}
template <typename T, int HD, int N, bool DROP>
__global__ __launch_bounds__(256) void graph_edge_fwd_kernel(const GraphAttnArgs a) {
  graph_edge_pass<T, HD, N, DROP, 0>(a);
}
template <typename T, int HD, int N, bool DROP>
__global__ __launch_bounds__(256) void graph_edge_dq_kernel(const GraphAttnArgs a) {
  graph_edge_pass<T, HD, N, DROP, 1>(a);
}
template <typename T, int HD, int N, bool DROP>
__global__ __launch_bounds__(256) void graph_edge_dkdv_kernel(const GraphAttnArgs a) {
  graph_edge_pass<T, HD, N, DROP, 2>(a);
}

// row_of[e] = the CSR row holding entry e (-1 for an entry no row covers);
// with `sym`, *sym = 1 (the query pass clears it when the CSR is not its own
// transpose).
__global__ void fill_minus_one_kernel(int* __restrict__ p, long n, int* __restrict__ sym) {
  if (sym && blockIdx.x == 0 && threadIdx.x == 0) *sym = 1;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) p[i] = -1;
}
// Per query token t, kRowLanes lanes: row_of over its row (entries strided
// over the lanes), and its descriptor.  With `sym` (one segment array, as
// many queries as keys): clears *sym unless the CSR equals its transpose as
// far as row t shows -- its bounds in order (row 0 from 0, the last row to
// nnz), its entries keys in [0, total_k) in ascending order, and each entry
// (t, x), the r-th of equal ones, matched by an r-th entry t in row x (a
// binary search there).  Over all rows this is a bijection between the
// entries (t, x) and (x, t) with multiplicity, i.e. indptr = t_indptr and
// indices = t_rows.  Each lane checks its own entries against their
// predecessors (order, and r from the run of equal ones before it), so a
// row's checks run side by side: the chain of dependent loads per lane is one
// entry's (with one thread per row it was the whole row's: 15.8 -> 7.6 us at
// 65,486 tokens of degree 4.6, the group's segment search included).
constexpr int kRowLanes = 8;

// seg_of(cu, nseg, t) by the kRowLanes lanes of one row (lane j of the group
// at bit offset `shift` of the wave's ballot): an 8-ary search, one dependent
// load per step instead of one per halving (wave_seg_of's method per group).
DEVI int group_seg_of(const int* __restrict__ cu, int nseg, int t, int j, int shift) {
  int base = 0, span = nseg;
  while (span > 1) {
    const int step = (span + kRowLanes - 1) / kRowLanes, end = base + span;
    const int s = base + j * step;
    const uint32_t m = (uint32_t)(__ballot(s < end && cu[s] <= t) >> shift) & ((1u << kRowLanes) - 1u);
    if (m == 0) break;   // cu[base] > t: only possible at base 0 (seg_of's answer as well)
    base += (31 - __builtin_clz(m)) * step;
    span = min(step, end - base);
  }
  return base;
}
__global__ __launch_bounds__(256) void query_rows_kernel(const int* __restrict__ indptr,
                                                         const int* __restrict__ indices, const int* __restrict__ cu_q,
                                                         const int* __restrict__ cu_k, int nseg, int total_q,
                                                         int total_k, int nnz, int* __restrict__ row_of,
                                                         int4* __restrict__ q_desc, int* __restrict__ sym) {
  const long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int t = (int)(g / kRowLanes), j = (int)(g % kRowLanes);
  if (t >= total_q) return;
  int pa, pb;
  csr_row(indptr, t, nnz, pa, pb);
  for (int p = pa + j; p < pb; p += kRowLanes) row_of[p] = t;
  const int sg = group_seg_of(cu_q, nseg, t, j, (int)(threadIdx.x & 63) - j);   // all lanes of the row
  if (j == 0) q_desc[t] = make_desc(cu_k, total_k, indptr, nnz, sg, t);
  if (!sym) return;
  const int ra = indptr[t], rb = indptr[t + 1];
  bool ok = ra >= 0 && ra <= rb && rb <= nnz && (t > 0 || ra == 0) && (t + 1 < total_q || rb == nnz);
  for (int p = pa + j; ok && p < pb; p += kRowLanes) {
    const int x = indices[p];
    if (x < 0 || x >= total_k || (p > pa && x < indices[p - 1])) {
      ok = false;
      break;
    }
    int rank = 0;   // equal entries right before p (in a sorted row: all the earlier equal ones)
    while (p - rank > pa && indices[p - rank - 1] == x) ++rank;
    int lo, hi;
    csr_row(indptr, x, nnz, lo, hi);
    const int end = hi;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (indices[mid] < t) lo = mid + 1;
      else hi = mid;
    }
    ok = lo + rank < end && indices[lo + rank] == t;
  }
  if (!ok) *sym = 0;
}
// Per entry p: t_rows[p] = row_of[t_perm[p]], the query row of each
// transposed entry, and the plan's copy of the indices; per key token t (the
// first total_k threads): its descriptor over the transposed CSR.
__global__ void key_rows_kernel(const int* __restrict__ t_perm, const int* __restrict__ row_of, int nnz,
                                int* __restrict__ t_rows, const int* __restrict__ indices,
                                int* __restrict__ indices_copy, const int* __restrict__ t_indptr,
                                const int* __restrict__ cu_q, const int* __restrict__ cu_k, int nseg, int total_q,
                                int total_k, int4* __restrict__ k_desc, const int* __restrict__ sym) {
  if (sym && *sym) return;   // symmetric: sym_copy_kernel writes the transpose
  for (long p = (long)blockIdx.x * blockDim.x + threadIdx.x; p < max(nnz, total_k);
       p += (long)gridDim.x * blockDim.x) {
    if (p < nnz) {
      t_rows[p] = row_of[t_perm[p]];
      if (indices_copy) indices_copy[p] = indices[p];
    }
    if (p < total_k) k_desc[p] = make_desc(cu_q, total_q, t_indptr, nnz, seg_of(cu_k, nseg, (int)p), (int)p);
  }
}

// A symmetric CSR (*sym set by the query pass) is its own transpose:
// t_indptr = indptr, t_rows = indices and, with one segment array, each key's
// descriptor is its query descriptor; plus the plan's copy of the indices.
__global__ void sym_copy_kernel(const int* __restrict__ sym, const int* __restrict__ indptr,
                                const int* __restrict__ indices, const int4* __restrict__ q_desc, int nnz,
                                int total_k, int* __restrict__ t_indptr, int* __restrict__ t_rows,
                                int4* __restrict__ k_desc, int* __restrict__ indices_copy) {
  if (!*sym) return;
  const long n = max((long)nnz, (long)total_k + 1);
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    if (i < nnz) {
      const int x = indices[i];
      t_rows[i] = x;
      if (indices_copy) indices_copy[i] = x;
    }
    if (i <= total_k) t_indptr[i] = indptr[i];
    if (i < total_k) k_desc[i] = q_desc[i];
  }
}

size_t al256(size_t x) { return (x + 255) & ~size_t(255); }

// Node plan (mask_b of ESA_MASK_NODE_PLAN): the CSR's indices [nnz] first (so
// the plan reads as the indices array), the transposed CSR t_indptr
// [total_k + 1] and t_rows [nnz], the token descriptors of the queries
// (q_desc [total_q]) and keys (k_desc [total_k]), then the build's scratch
// (row_of, t_perm and the CSR sort's workspace).  The per-call backward lays
// the same arrays and scratch out in its workspace.
struct NodePlan { size_t indices, t_indptr, t_rows, q_desc, k_desc, row_of, t_perm, sym, csr, csr_bytes, total; };

int node_plan_layout(int total_q, int total_k, int nnz, NodePlan& w) {
  w = NodePlan{};
  const int rc = esa_csr_workspace_size(nnz, total_k, &w.csr_bytes);
  if (rc) return rc;
  size_t off = 0;
  w.indices = off; off += al256((size_t)nnz * 4 + 4);
  w.t_indptr = off; off += al256(((size_t)total_k + 1) * 4);
  w.t_rows = off; off += al256((size_t)nnz * 4 + 4);
  w.q_desc = off; off += al256((size_t)total_q * 16 + 16);
  w.k_desc = off; off += al256((size_t)total_k * 16 + 16);
  w.row_of = off; off += al256((size_t)nnz * 4 + 4);
  w.t_perm = off; off += al256((size_t)nnz * 4 + 4);
  w.sym = off; off += 256;
  w.csr = off; off += al256(w.csr_bytes);
  w.total = off;
  return ESA_OK;
}

unsigned grid_of(long n) { const long b = (n + 255) / 256; return (unsigned)(b < 1 ? 1 : b < 4096 ? b : 4096); }

// The transposed CSR of (indptr, indices) and both sides' token descriptors
// into base's NodePlan layout; copy_indices: also the plan's copy of the
// indices.
int build_transposed(const int* indptr, const int* indices, const int* cu_q, const int* cu_k, int nseg,
                     int total_q, int total_k, int nnz, char* base, const NodePlan& w, bool copy_indices,
                     hipStream_t st) {
  int* row_of = reinterpret_cast<int*>(base + w.row_of);
  int* t_perm = reinterpret_cast<int*>(base + w.t_perm);
  int* t_indptr = reinterpret_cast<int*>(base + w.t_indptr);
  int* t_rows = reinterpret_cast<int*>(base + w.t_rows);
  int4* q_desc = reinterpret_cast<int4*>(base + w.q_desc);
  int4* k_desc = reinterpret_cast<int4*>(base + w.k_desc);
  int* indices_copy = copy_indices ? reinterpret_cast<int*>(base + w.indices) : nullptr;
  // One segment array and as many queries as keys: the query pass tests whether the CSR is its own
  // transpose (a device flag, no host synchronisation); if it is, the sort's and the key pass's launches
  // return at once and sym_copy_kernel copies the CSR into the transposed sections.
  int* sym = (cu_q == cu_k && total_q == total_k && nnz > 0) ? reinterpret_cast<int*>(base + w.sym) : nullptr;
  if (nnz > 0) {
    hipLaunchKernelGGL(fill_minus_one_kernel, dim3(grid_of(nnz)), dim3(256), 0, st, row_of, (long)nnz, sym);
    ESA_LAUNCH_CHECK();
  }
  if (total_q > 0) {
    hipLaunchKernelGGL(query_rows_kernel, dim3((unsigned)(((long)total_q * kRowLanes + 255) / 256)), dim3(256), 0, st,
                       indptr, indices, cu_q, cu_k, nseg, total_q, total_k, nnz, row_of, q_desc, sym);
    ESA_LAUNCH_CHECK();
  }
  int rc = csr_build_impl(indices, nnz, total_k, t_indptr, t_perm, base + w.csr, w.csr_bytes, st, sym);
  if (rc) return rc;
  if (nnz > 0 || total_k > 0) {
    hipLaunchKernelGGL(key_rows_kernel, dim3(grid_of(nnz > total_k ? nnz : total_k)), dim3(256), 0, st, t_perm,
                       row_of, nnz, t_rows, indices, indices_copy, t_indptr, cu_q, cu_k, nseg, total_q, total_k,
                       k_desc, sym);
    ESA_LAUNCH_CHECK();
  }
  if (sym) {
    hipLaunchKernelGGL(sym_copy_kernel, dim3(grid_of(nnz > total_k + 1 ? nnz : total_k + 1)), dim3(256), 0, st,
                       sym, indptr, indices, q_desc, nnz, total_k, t_indptr, t_rows, k_desc, indices_copy);
    ESA_LAUNCH_CHECK();
  }
  return ESA_OK;
}

struct GraphWs { size_t dsum, plan, total; };

int graph_ws(int total_q, int total_k, int heads, int nnz, bool backward, bool planned, GraphWs& w) {
  w = GraphWs{};
  if (!backward) return ESA_OK;
  size_t off = 0;
  w.dsum = off; off += al256((size_t)heads * total_q * 4);
  if (!planned) {
    NodePlan np;
    const int rc = node_plan_layout(total_q, total_k, nnz, np);
    if (rc) return rc;
    w.plan = off; off += np.total;
  }
  w.total = off;
  return ESA_OK;
}

unsigned token_blocks(int tokens) { return (unsigned)((tokens + 3) / 4); }

}  // namespace

int graph_attn_workspace_size(int total_q, int total_k, int heads, int nnz, bool backward, bool planned,
                              size_t* bytes) {
  GraphWs w;
  const int rc = graph_ws(total_q, total_k, heads, nnz, backward, planned, w);
  if (rc) return rc;
  *bytes = w.total;
  return ESA_OK;
}

int graph_node_plan_size(int total_q, int total_k, int nnz, size_t* bytes) {
  NodePlan w;
  const int rc = node_plan_layout(total_q, total_k, nnz, w);
  if (rc) return rc;
  *bytes = w.total;
  return ESA_OK;
}

int graph_node_plan_sections(int total_q, int total_k, int nnz, size_t offsets[5]) {
  NodePlan w;
  const int rc = node_plan_layout(total_q, total_k, nnz, w);
  if (rc) return rc;
  offsets[0] = w.indices;
  offsets[1] = w.t_indptr;
  offsets[2] = w.t_rows;
  offsets[3] = w.q_desc;
  offsets[4] = w.k_desc;
  return ESA_OK;
}

int graph_node_plan_build(const int* indptr, const int* indices, const int* cu_q, const int* cu_k, int nseg,
                          int total_q, int total_k, int nnz, void* plan, size_t plan_bytes, hipStream_t st) {
  NodePlan w;
  int rc = node_plan_layout(total_q, total_k, nnz, w);
  if (rc) return rc;
  if (plan_bytes < w.total) return ESA_ERR_WORKSPACE;
  return build_transposed(indptr, indices, cu_q, cu_k, nseg, total_q, total_k, nnz, static_cast<char*>(plan), w,
                          true, st);
}

namespace {

// Dims per lane: 8 where a wave then needs fewer passes over the heads than
// with 4 (never at head dim 24).
int dims_per_lane(int heads, int head_dim) {
  if (head_dim == 24) return 4;
  auto passes = [&](int n) { const int hpp = 64 / (head_dim / n); return (heads + hpp - 1) / hpp; };
  return passes(8) < passes(4) ? 8 : 4;
}

// Launches KERNEL<T, HD, N, DROP> for the call's dtype, head dim, dims per
// lane and dropout.
#define ESA_GRAPH_LAUNCH_N(KERNEL, T, D, hd, n, grid, st, a)                                      \
  do {                                                                                            \
    if (n == 8) {                                                                                 \
      if (hd == 16) hipLaunchKernelGGL((KERNEL<T, 16, 8, D>), grid, dim3(256), 0, st, a);         \
      else if (hd == 32) hipLaunchKernelGGL((KERNEL<T, 32, 8, D>), grid, dim3(256), 0, st, a);    \
      else hipLaunchKernelGGL((KERNEL<T, 64, 8, D>), grid, dim3(256), 0, st, a);                  \
    } else {                                                                                      \
      if (hd == 16) hipLaunchKernelGGL((KERNEL<T, 16, 4, D>), grid, dim3(256), 0, st, a);         \
      else if (hd == 24) hipLaunchKernelGGL((KERNEL<T, 24, 4, D>), grid, dim3(256), 0, st, a);    \
      else if (hd == 32) hipLaunchKernelGGL((KERNEL<T, 32, 4, D>), grid, dim3(256), 0, st, a);    \
      else hipLaunchKernelGGL((KERNEL<T, 64, 4, D>), grid, dim3(256), 0, st, a);                  \
    }                                                                                             \
  } while (0)
#define ESA_GRAPH_LAUNCH(KERNEL, dtype, hd, grid, st, a)                                          \
  do {                                                                                            \
    const int n_ = dims_per_lane(a.heads, hd);                                                    \
    if (dtype == ESA_F32) {                                                                       \
      if (a.dropout) ESA_GRAPH_LAUNCH_N(KERNEL, float, true, hd, n_, grid, st, a);                \
      else ESA_GRAPH_LAUNCH_N(KERNEL, float, false, hd, n_, grid, st, a);                         \
    } else {                                                                                      \
      if (a.dropout) ESA_GRAPH_LAUNCH_N(KERNEL, bf16, true, hd, n_, grid, st, a);                 \
      else ESA_GRAPH_LAUNCH_N(KERNEL, bf16, false, hd, n_, grid, st, a);                          \
    }                                                                                             \
  } while (0)

}  // namespace

int graph_attn_fwd(GraphAttnArgs a, int dtype, const void* plan, hipStream_t st) {
  if (a.total_q == 0) return ESA_OK;
  if (!graph_head_dim_ok(a.head_dim)) return ESA_ERR_HEAD_DIM;
  a.q_desc = nullptr;
  if (plan) {
    NodePlan np;
    const int rc = node_plan_layout(a.total_q, a.total_k, a.nnz, np);
    if (rc) return rc;
    a.q_desc = reinterpret_cast<const int4*>(static_cast<const char*>(plan) + np.q_desc);
  }
  const dim3 grid(token_blocks(a.total_q));
  ESA_TIMED(esa_profile::kGraphFwd, st, ESA_GRAPH_LAUNCH(graph_attn_fwd_kernel, dtype, a.head_dim, grid, st, a));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

int graph_attn_bwd(GraphAttnArgs a, int dtype, const void* plan, void* workspace, size_t workspace_bytes,
                   hipStream_t st) {
  if (!graph_head_dim_ok(a.head_dim)) return ESA_ERR_HEAD_DIM;
  GraphWs w;
  int rc = graph_ws(a.total_q, a.total_k, a.heads, a.nnz, true, plan != nullptr, w);
  if (rc) return rc;
  if (workspace_bytes < w.total) return ESA_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  a.dsum = reinterpret_cast<float*>(ws + w.dsum);
  NodePlan np;
  if ((rc = node_plan_layout(a.total_q, a.total_k, a.nnz, np))) return rc;
  const char* tbase;
  if (plan) {
    tbase = static_cast<const char*>(plan);
  } else {
    if ((rc = build_transposed(a.indptr, a.indices, a.cu_q, a.cu_k, a.nseg, a.total_q, a.total_k, a.nnz,
                               ws + w.plan, np, false, st)))
      return rc;
    tbase = ws + w.plan;
  }
  a.t_indptr = reinterpret_cast<const int*>(tbase + np.t_indptr);
  a.t_rows = reinterpret_cast<const int*>(tbase + np.t_rows);
  a.q_desc = reinterpret_cast<const int4*>(tbase + np.q_desc);
  a.k_desc = reinterpret_cast<const int4*>(tbase + np.k_desc);
  if (a.total_q > 0) {
    ESA_TIMED(esa_profile::kGraphDq, st,
              ESA_GRAPH_LAUNCH(graph_attn_dq_kernel, dtype, a.head_dim, dim3(token_blocks(a.total_q)), st, a));
    ESA_LAUNCH_CHECK();
  }
  if (a.total_k > 0) {
    ESA_TIMED(esa_profile::kGraphDkdv, st,
              ESA_GRAPH_LAUNCH(graph_attn_dkdv_kernel, dtype, a.head_dim, dim3(token_blocks(a.total_k)), st, a));
    ESA_LAUNCH_CHECK();
  }
  return ESA_OK;
}

int graph_edge_attn_fwd(GraphAttnArgs a, int dtype, hipStream_t st) {
  if (a.total_q == 0) return ESA_OK;
  if (!graph_head_dim_ok(a.head_dim)) return ESA_ERR_HEAD_DIM;
  ESA_TIMED(esa_profile::kAttnFwdMasked, st,
            ESA_GRAPH_LAUNCH(graph_edge_fwd_kernel, dtype, a.head_dim, dim3(token_blocks(a.total_q)), st, a));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

int graph_edge_attn_bwd(GraphAttnArgs a, int dtype, void* workspace, size_t workspace_bytes, hipStream_t st) {
  if (!graph_head_dim_ok(a.head_dim)) return ESA_ERR_HEAD_DIM;
  GraphWs w;
  int rc = graph_ws(a.total_q, a.total_k, a.heads, 0, true, true, w);
  if (rc) return rc;
  if (workspace_bytes < w.total) return ESA_ERR_WORKSPACE;
  a.dsum = reinterpret_cast<float*>(static_cast<char*>(workspace) + w.dsum);
  if (a.total_q > 0) {
    ESA_TIMED(esa_profile::kAttnBwdDqMasked, st,
              ESA_GRAPH_LAUNCH(graph_edge_dq_kernel, dtype, a.head_dim, dim3(token_blocks(a.total_q)), st, a));
    ESA_LAUNCH_CHECK();
  }
  if (a.total_k > 0) {
    ESA_TIMED(esa_profile::kAttnBwdDkdvMasked, st,
              ESA_GRAPH_LAUNCH(graph_edge_dkdv_kernel, dtype, a.head_dim, dim3(token_blocks(a.total_k)), st, a));
    ESA_LAUNCH_CHECK();
  }
  return ESA_OK;
}
