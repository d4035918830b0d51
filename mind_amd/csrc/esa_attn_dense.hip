// Segment-tiled dense attention (no mask), bf16 operands, fp32 softmax, on gfx950.
//
// Semantics: flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, ...,
// causal=False, dropout 0) as called at esa/mha_flash_varlen.py:177-184.
//
// Work items are 128-token groups cut from each segment on its own, so a
// block never straddles two segments: its four waves own four consecutive
// 32-token tiles of one segment and walk the same partner range, and only
// the last, partial partner tile of a segment needs a per-element test.  A
// per-call plan (one block per direction) lists the groups longest partner
// range first.  Partner tokens are staged 64 at a time (two 32-token tiles)
// into double-buffered LDS with one barrier per stage and loads two stages
// ahead; every wave stages 16 tokens of both operands of the stage (lanes
// 0..31 the first tensor, 32..63 the second), transposing in the LDS write
// where an MFMA operand needs the token dimension contiguous.  Blocks of one
// head share an XCD (head = blockIdx % heads) and its L2.
//
// Register layouts follow esa_attn_tiles.h (v_mfma_f32_32x32x16_bf16,
// head_dim = the MFMA K of 16).  The softmax scale c = scale * log2(e) rides
// in the MFMAs instead of a VALU multiply per score: the operand that is
// fixed per lane for the whole walk (q in the forward and dQ pass, k in the
// dK/dV pass) is multiplied by c once and split into bf16 hi + lo halves,
// two MFMAs accumulate hi and lo, and the log-sum-exp offset enters as the
// accumulator seed (dQ) or through a row-statistic MFMA (dK/dV), so every
// probability is a bare exp2 of an MFMA result.
#include "esa_attn_tiles.h"
#include "esa_attn_dense.h"
#include "esa_profile.h"
#include "../../include/esa_hip.h"

namespace {

constexpr int kStageTok = 64;      // partner tokens per staging step (two tiles)

// Build-time tuning: minimum waves per SIMD each kernel is compiled for
// (0 = compiler's choice).
#ifndef ESA_DENSE_WAVES_FWD
#define ESA_DENSE_WAVES_FWD 4
#endif
#ifndef ESA_DENSE_WAVES_DQ
#define ESA_DENSE_WAVES_DQ 5
#endif
#ifndef ESA_DENSE_WAVES_DKDV
#define ESA_DENSE_WAVES_DKDV 0
#endif
#define ESA_WAVES_ATTR(n) __attribute__((amdgpu_waves_per_eu(n > 0 ? n : 1)))

struct DenseArgs {
  const bf16* q; const bf16* k; const bf16* v; const bf16* out; const bf16* dout;
  const float2* aux;           // dK/dV: per (head, query) {-LSE2, -D}, [H][tq_pad]
  float2* aux_out;             // dQ: writes aux for its queries (dQ runs first)
  const float* lse;            // dQ: [H][Tq] natural log
  const float* knorm;          // forward: max |k| per (head, global 32-token tile), [H][tk_tiles]
  int tk_tiles;
  const int4* groups;          // (outer begin, outer segment end, inner begin, inner end)
  const int* count;            // number of groups
  int total_q, total_k, heads, tq_pad;
  float c, scale;              // c = scale * log2(e)
  bf16* o; float* lse_out; bf16* dq; bf16* dk; bf16* dv;
};

// ------------------------------------------------------------------ block mapping
// Hardware block b runs on XCD b % 8, and each XCD has its own L2.  A 128-byte
// line of a [T][H][16] bf16 tensor holds one token's rows of four
// consecutive heads ("a line group").  For H = 4, 8, 16 or 32 the blocks are
// mapped so that each XCD serves the four heads of one line group: with
// lines = H / 4 groups, r = 8 / lines XCDs share one line group and each
// takes every r-th work item (H = 32: one XCD per line group, each line
// fetched by one L2; H = 16: two).  Other head counts use head = b % heads.
#ifndef ESA_DENSE_XCD_LINES
#define ESA_DENSE_XCD_LINES 1
#endif

DEVI bool xcd_lines(int H) { return ESA_DENSE_XCD_LINES && (H == 4 || H == 8 || H == 16 || H == 32); }

DEVI void block_item_head(int H, int& item, int& head) {
  const int b = blockIdx.x;
  if (xcd_lines(H)) {
    const int r = 32 / H;   // XCDs per line group: 8 / (H / 4)
    const int xcd = b & 7, slot = b >> 3;
    head = 4 * (xcd / r) + (slot & 3);
    item = r * (slot >> 2) + xcd % r;
  } else {
    item = b / H;
    head = b - item * H;
  }
}

unsigned group_blocks(int groups, int H) {
  if (ESA_DENSE_XCD_LINES && (H == 4 || H == 8 || H == 16 || H == 32)) {
    const int r = 32 / H;
    return (unsigned)(32 * ((groups + r - 1) / r));   // 8 XCDs x 4 heads x ceil(groups / r) items
  }
  return (unsigned)(groups * H);
}

// ------------------------------------------------------------------ staging

// This lane's 16-byte chunk of a stage: lanes 0..31 read tensor A, 32..63
// tensor B, one global load with a per-lane address (a single instruction,
// so a stage's load is waited for on its own and the next stage's load
// stays in flight).  The token is clamped into the tensor: a row past the
// segment is masked in the compute whatever it holds.
DEVI i32x4 stage_chunk(const bf16* __restrict__ a, const bf16* __restrict__ b, int token, int total, int H,
                       int head, int hf, int lane) {
  const bf16* base = lane < 32 ? a : b;
  const int t = min(token, total - 1);
  return *reinterpret_cast<const i32x4*>(base + ((size_t)t * H + head) * kHd + 8 * hf);
}
constexpr uint32_t kNoLoad = 0xFFFFFFF0u;   // buffer offset past any range: the load returns zeros

// Stage loads run kStageDepth stages ahead of the compute through a ring of
// register sets, two LDS buffers, one barrier per stage: while stage s is
// computed, stages s + 1 .. s + kStageDepth are in flight or held, so the
// global latency of a stage is hidden behind kStageDepth - 1 stages of
// compute.  gload(st) returns this lane's staging registers, lstore(buf, r)
// writes them, compute(buf, st) consumes a staged stage.  Past the end the
// loads re-read the last stage and are never stored; the loop is unrolled
// by the depth so the ring's registers never move.
#ifndef ESA_STAGE_DEPTH
#define ESA_STAGE_DEPTH 2
#endif
constexpr int kStageDepth = ESA_STAGE_DEPTH;
static_assert(kStageDepth >= 2 && kStageDepth % 2 == 0, "stage ring depth must be even");

template <class Load, class Store, class Compute>
DEVI void stage_walk(int n_stages, Load gload, Store lstore, Compute compute) {
  if (n_stages <= 0) return;
  decltype(gload(0)) r[kStageDepth];
#pragma unroll
  for (int i = 0; i < kStageDepth; ++i) r[i] = gload(min(i, n_stages - 1));
  lstore(0, r[0]);
  __syncthreads();
  for (int st = 0; st < n_stages; st += kStageDepth) {
#pragma unroll
    for (int i = 0; i < kStageDepth; ++i) {
      const int s = st + i;   // in LDS buffer i & 1; r[i] held it and is free
      if (s >= n_stages) return;
      r[i] = gload(min(s + kStageDepth, n_stages - 1));
      compute(i & 1, s);
      if (s + 1 < n_stages) lstore((i + 1) & 1, r[(i + 1) % kStageDepth]);
      __syncthreads();
    }
  }
}

struct Stage2 { i32x4 a, b; };

// ---- staging layouts of the 16x16 backward kernels (LDS bank-conflict free
// for their reads and writes on gfx950).  Lane l of wave w stages dims
// 8 h .. 8 h + 7, h = (l >> 4) & 1, of stage token 16 w + (l & 15), so 16
// consecutive lanes write 256 contiguous bytes.
DEVI int split_tok(int wave, int lane) { return 16 * wave + (lane & 15); }
DEVI int split_half(int lane) { return (lane >> 4) & 1; }

// Staged rows split by dims half (esa_attn_tiles.h), one stage of
// kStageTok tokens per buffer.
constexpr int kHalfRows = kStageTok * 8;   // bf16 per dims half
constexpr int kSplitRows = 2 * kHalfRows;  // bf16 per staged stage

// The two tiles of a staged stage, each reading its LDS operands right
// before its compute (reading both tiles' operands first costs more in
// registers and occupancy than the LDS latency it hides).
template <class Ops, class Tile>
DEVI void stage_tiles(int buf, int st, int n_tiles, Ops ops, Tile tile, int t0) {
  tile(ops(buf, 0), t0);
  if (2 * st + 1 < n_tiles) tile(ops(buf, 1), t0 + kTile);
}

// ------------------------------------------------------------------ forward
// Each wave owns kFwdTiles consecutive 32-query tiles: every K row and V^T
// operand read from LDS feeds that many independent score / softmax / PV
// chains, so one chain's exponentials overlap another's MFMAs.

#ifndef ESA_FWD_TILES
#define ESA_FWD_TILES 2
#endif
constexpr int kFwdTiles = ESA_FWD_TILES;
constexpr int kFwdGroup = kWaves * kTile * kFwdTiles;   // queries per block

__global__ __launch_bounds__(256) ESA_WAVES_ATTR(ESA_DENSE_WAVES_FWD) void dense_fwd_kernel(const DenseArgs a) {
  constexpr int T = kFwdTiles;
  __shared__ __align__(16) bf16 sK[2][kSplitRows];   // K rows split by dims half
  __shared__ __align__(16) bf16 sV[2][kSplitRows];   // V rows split by dims half
  __shared__ __align__(16) bf16 sOnes[4];             // the ones rows of [V^T ; 1]
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5, c16 = lane & 15, grp = lane >> 4;
  const int H = a.heads;
  int item, head;
  block_item_head(H, item, head);
  if (item >= *a.count) return;
  const int4 g = a.groups[item];

  if (tid < 4) sOnes[tid] = (bf16)1.f;   // visible after the walk's first barrier
  const int o0 = g.x + wave * kTile * T;
  int t[T];
  bool valid[T], active[T];
  bf16x8 qh[T], ql[T];
  float bnd = 0.f;
  float km = 0.f;
  for (int tt = (g.z >> 5) + lane; tt < ((g.w + kTile - 1) >> 5); tt += 64)
    km = fmaxf(km, a.knorm[(size_t)head * a.tk_tiles + tt]);
  km = wave_max(km);
#pragma unroll
  for (int u = 0; u < T; ++u) {
    active[u] = o0 + u * kTile < g.y;
    t[u] = o0 + u * kTile + col;
    valid[u] = t[u] < g.y;
    const int tc = valid[u] ? t[u] : g.x;
    const bf16x8 qf = *reinterpret_cast<const bf16x8*>(a.q + ((size_t)tc * H + head) * kHd + 8 * half);
    float qq = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) qq = fmaf((float)qf[e], (float)qf[e], qq);
    qq += __shfl_xor(qq, 32);
    bnd = fmaxf(bnd, valid[u] ? a.c * sqrtf(qq) * km : 0.f);   // bound b = c |q| max|k| over the segment's keys
    split_scaled(qf, a.c, qh[u], ql[u]);
  }
  const bool any_active = active[0];
  const bool fixed_ref = __builtin_amdgcn_readfirstlane((int)(wave_max(bnd) <= kStaticBound)) != 0;

  const int n_tiles = (g.w - g.z + kTile - 1) >> 5;
  const int n_stages = (n_tiles + 1) >> 1;
  const int tok = split_tok(wave, lane), hs = split_half(lane);
  auto gload = [&](int st) { return stage_chunk(a.k, a.v, g.z + st * kStageTok + tok, a.total_k, H, head, hs, lane); };
  auto lstore = [&](int buf, i32x4 r) { put_half<kHalfRows>(lane < 32 ? sK[buf] : sV[buf], tok, hs, r); };

  float m_run[T];
  f32x16 acc[T];
#pragma unroll
  for (int u = 0; u < T; ++u) {
    m_run[u] = fixed_ref ? 0.f : -INFINITY;
    acc[u] = f32x16{};
  }
  const f32x16 zero = {};
  auto run = [&](auto online_tag) {
    constexpr bool ONLINE = decltype(online_tag)::value;
    auto k_rows = [&](int buf, int j) { return half_row8<kHalfRows>(sK[buf], 32 * j + kperm(col), half); };
    auto scores = [&](const bf16x8& kr, int u) { return mfma32(kr, ql[u], mfma32(kr, qh[u], zero)); };
    // Softmax of query tile u's scores s against one key tile (keys k0..),
    // then P V into acc[u].
    auto softmax_pv = [&](int u, f32x16 s, int k0, const bf16x8& vt0, const bf16x8& vt1) {
      if (k0 + kTile > g.w) {   // the segment's last, partial key tile
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = k0 + row_local(r, half) < g.w ? s[r] : -INFINITY;
      }
      float p[16];
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
        const float m_use = m_run[u] == -INFINITY ? 0.f : m_run[u];
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = fast_exp2(s[r] - m_use);
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = fast_exp2(s[r]);
      }
      acc[u] = mfma32(vt0, cvt8(p), acc[u]);
      acc[u] = mfma32(vt1, cvt8(p + 8), acc[u]);
    };
    // LDS operands of key tile j: K rows and the two [V^T ; 1] operands.
    struct Ops { bf16x8 kr, vt0, vt1; };
    auto ops = [&](int buf, int j) {
      Ops o;
      o.kr = k_rows(buf, j);
      tr_rows32<kHalfRows>(sV[buf], 32 * j, sOnes, c16, grp, o.vt0, o.vt1);
      return o;
    };
    // One key tile: the score MFMAs of all query tiles first, then each
    // query tile's softmax and P V.
    auto tile = [&](const Ops& o, int k0) {
      f32x16 s[T];
#pragma unroll
      for (int u = 0; u < T; ++u) s[u] = scores(o.kr, u);
#pragma unroll
      for (int u = 0; u < T; ++u)
        if (u == 0 || active[u]) softmax_pv(u, s[u], k0, o.vt0, o.vt1);   // active[u]: wave-uniform
    };
    stage_walk(n_stages, gload, lstore, [&](int buf, int st) {
      if (!any_active) return;
      stage_tiles(buf, st, n_tiles, ops, tile, g.z + st * kStageTok);
    });
  };
  if (fixed_ref)
    run(std::integral_constant<bool, false>{});
  else
    run(std::integral_constant<bool, true>{});
#pragma unroll
  for (int u = 0; u < T; ++u) {
    if (!valid[u]) continue;
    const float l = acc[u][8];   // a ones row of [V^T; 1] P^T: the softmax row sum
    store_rows8(a.o + ((size_t)t[u] * H + head) * kHd, acc[u], l > 0.f ? 1.f / l : 0.f, half);
    if (half == 0)
      a.lse_out[(size_t)head * a.total_q + t[u]] = l > 0.f ? (m_run[u] + fast_log2(l)) * kLn2 : -INFINITY;
  }
}

// ------------------------------------------------------------------ dQ pass
// One wave = kDqTiles tiles of 32 queries; dQ = scale * sum_k P (dP - D) k
// in 16x16 blocks (esa_attn_tiles.h): S'^T = K (c q)^T - LSE2 by one
// mfma16k32 per (key block, query block) with the hi / lo halves of c q in
// its K slots and -LSE2 as the accumulator seed, dP^T - D by one mfma16k16
// seeded with -D, P = exp2(S'), and dQ^T += K^T dS^T by one mfma16k32 per
// query block over a key tile's 32 keys.  Every K, V and K^T operand read
// from LDS feeds all of the wave's query blocks.

#ifndef ESA_DQ_TILES
#define ESA_DQ_TILES 1
#endif
constexpr int kDqTiles = ESA_DQ_TILES;
constexpr int kDqGroup = kWaves * kTile * kDqTiles;   // queries per block

__global__ __launch_bounds__(256) ESA_WAVES_ATTR(ESA_DENSE_WAVES_DQ) void dense_dq_kernel(const DenseArgs a) {
  constexpr int T = kDqTiles;
  __shared__ __align__(16) bf16 sK[2][kSplitRows];   // K rows split by dims half
  __shared__ __align__(16) bf16 sV[2][kSplitRows];   // V rows split by dims half
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, grp = lane >> 4;
  const int H = a.heads;
  int item, head;
  block_item_head(H, item, head);
  if (item >= *a.count) return;
  const int4 g = a.groups[item];

  const int o0 = g.x + wave * kTile * T;
  bool active[T];
  bf16x8 qs[T][2];     // B of the score MFMA: scaled hi / lo halves of q
  bf16x4 ob[T][2];     // B of the dP MFMA: dO dims 4 grp..+3
  f32x4 cl[T][2], cd[T][2];
#pragma unroll
  for (int u = 0; u < T; ++u) {
    active[u] = o0 + u * kTile < g.y;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int t = o0 + u * kTile + 16 * qb + c16;
      const int tc = t < g.y ? t : g.x;
      const size_t row = ((size_t)tc * H + head) * kHd;
      const bf16x8 d0 = *reinterpret_cast<const bf16x8*>(a.dout + row);
      const bf16x8 d1 = *reinterpret_cast<const bf16x8*>(a.dout + row + 8);
      const bf16x8 p0 = *reinterpret_cast<const bf16x8*>(a.out + row);
      const bf16x8 p1 = *reinterpret_cast<const bf16x8*>(a.out + row + 8);
      float dsum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) dsum = fmaf((float)d0[e], (float)p0[e], dsum);
#pragma unroll
      for (int e = 0; e < 8; ++e) dsum = fmaf((float)d1[e], (float)p1[e], dsum);
      qs[u][qb] = scaled_half(*reinterpret_cast<const bf16x8*>(a.q + row + 8 * (grp & 1)), a.c, grp >= 2);
      ob[u][qb] = *reinterpret_cast<const bf16x4*>(a.dout + row + 4 * grp);
      const float lq = a.lse[(size_t)head * a.total_q + tc];
      cl[u][qb] = splat4(lq == -INFINITY ? -INFINITY : -lq * kLog2e);   // seed of S': -LSE2
      cd[u][qb] = splat4(-dsum);                                        // seed of dP: -D
      // the dK/dV pass's row statistics of this query (rows without keys: a finite -LSE2 so that P = 0)
      if (grp == 0 && t < g.y)
        a.aux_out[(size_t)head * a.tq_pad + t] = make_float2(lq == -INFINITY ? kDeadRow : -lq * kLog2e, -dsum);
    }
  }

  const int n_tiles = (g.w - g.z + kTile - 1) >> 5;
  const int n_stages = (n_tiles + 1) >> 1;
  const int tok = split_tok(wave, lane), hs = split_half(lane);
  auto gload = [&](int st) { return stage_chunk(a.k, a.v, g.z + st * kStageTok + tok, a.total_k, H, head, hs, lane); };
  auto lstore = [&](int buf, i32x4 r) {
    put_half<kHalfRows>(lane < 32 ? sK[buf] : sV[buf], tok, hs, r);
  };

  f32x4 acc[T][2];
#pragma unroll
  for (int u = 0; u < T; ++u) acc[u][0] = acc[u][1] = f32x4{};
  // One key tile of the staged pair: every block's score and dP MFMAs
  // first, then each query block's exponentials and dS K.
  struct Ops { bf16x8 ka[2], kt; bf16x4 va[2]; };
  auto ops = [&](int buf, int j) {
    Ops o;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      o.ka[kb] = half_row8<kHalfRows>(sK[buf], 32 * j + 16 * kb + c16, grp & 1);
      o.va[kb] = half_row4<kHalfRows>(sV[buf], 32 * j + 16 * kb + c16, grp);
    }
    o.kt = tr_operand<kHalfRows>(sK[buf], 32 * j, c16, grp);
    return o;
  };
  auto tile = [&](const Ops& o, int k0) {
    const bf16x8* ka = o.ka;
    const bf16x4* va = o.va;
    const bf16x8& kt = o.kt;
    f32x4 s[T][2][2], dp[T][2][2];   // [u][query block][key block]
#pragma unroll
    for (int u = 0; u < T; ++u)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          s[u][qb][kb] = mfma16k32(ka[kb], qs[u][qb], cl[u][qb]);
          dp[u][qb][kb] = mfma16k16(va[kb], ob[u][qb], cd[u][qb]);
        }
    if (k0 + kTile > g.w) {   // the segment's last, partial key tile
#pragma unroll
      for (int u = 0; u < T; ++u)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              s[u][qb][kb][e] = k0 + 16 * kb + 4 * grp + e < g.w ? s[u][qb][kb][e] : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < T; ++u) {
      if (u > 0 && !active[u]) continue;   // wave-uniform
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        f32x4 ds[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e) ds[kb][e] = fast_exp2(s[u][qb][kb][e]) * dp[u][qb][kb][e];
        acc[u][qb] = mfma16k32(kt, cvt4x2(ds[0], ds[1]), acc[u][qb]);
      }
    }
  };
  stage_walk(n_stages, gload, lstore, [&](int buf, int st) {
    if (!active[0]) return;
    stage_tiles(buf, st, n_tiles, ops, tile, g.z + st * kStageTok);
  });
#pragma unroll
  for (int u = 0; u < T; ++u)
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int t = o0 + u * kTile + 16 * qb + c16;
      if (t < g.y) store_dims4(a.dq + ((size_t)t * H + head) * kHd, acc[u][qb], a.scale, grp);
    }
}

// ------------------------------------------------------------------ dK/dV pass
// One wave = kDkdvTiles tiles of 32 keys; rows are queries, in 16x16 blocks
// (esa_attn_tiles.h): S' = Q (c k)^T - LSE2 by one mfma16k32 per (query
// block, key block) with the hi / lo halves of c k in its K slots, dP - D by
// one mfma16k16; the row statistics -LSE2 and -D are fp32 accumulator
// seeds read from LDS (four consecutive queries per lane group).  dV^T +=
// dO^T P^T and dK^T += Q^T dS^T by one mfma16k32 each per key block over a
// query tile's 32 queries.  Every Q, dO, Q^T, dO^T and statistic read from
// LDS feeds all of the wave's key blocks.

#ifndef ESA_DKDV_TILES
#define ESA_DKDV_TILES 1
#endif
constexpr int kDkdvTiles = ESA_DKDV_TILES;
constexpr int kDkdvGroup = kWaves * kTile * kDkdvTiles;   // keys per block

__global__ __launch_bounds__(256) ESA_WAVES_ATTR(ESA_DENSE_WAVES_DKDV) void dense_dkdv_kernel(const DenseArgs a) {
  constexpr int T = kDkdvTiles;
  __shared__ __align__(16) bf16 sQ[2][kSplitRows];     // rows split by dims half
  __shared__ __align__(16) bf16 sDO[2][kSplitRows];
  __shared__ __align__(16) float sLse[2][kStageTok];      // -LSE2 per query
  __shared__ __align__(16) float sDel[2][kStageTok];      // -D per query
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, grp = lane >> 4;
  const int H = a.heads;
  int item, head;
  block_item_head(H, item, head);
  if (item >= *a.count) return;
  const int4 g = a.groups[item];   // outer = keys, inner = queries

  const int o0 = g.x + wave * kTile * T;
  bool active[T];
  bf16x8 ks[T][2];     // B of the score MFMA: scaled hi / lo halves of k
  bf16x4 vb[T][2];     // B of the dP MFMA: v dims 4 grp..+3
#pragma unroll
  for (int u = 0; u < T; ++u) {
    active[u] = o0 + u * kTile < g.y;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int t = o0 + u * kTile + 16 * kb + c16;
      const int tc = t < g.y ? t : g.x;
      const size_t row = ((size_t)tc * H + head) * kHd;
      ks[u][kb] = scaled_half(*reinterpret_cast<const bf16x8*>(a.k + row + 8 * (grp & 1)), a.c, grp >= 2);
      vb[u][kb] = *reinterpret_cast<const bf16x4*>(a.v + row + 4 * grp);
    }
  }

  const int n_tiles = (g.w - g.z + kTile - 1) >> 5;
  const int n_stages = (n_tiles + 1) >> 1;
  const rsrc_t rx = make_rsrc(a.aux + (size_t)head * a.tq_pad, (uint32_t)a.tq_pad * 8u);
  const int tok = split_tok(wave, lane), hs = split_half(lane);
  // row statistics: lanes 0..7 of wave w fetch queries 16w .. 16w+15 (two 8-byte records per lane)
  const uint32_t aux0 = lane < 8 ? (uint32_t)(g.z + 16 * wave + 2 * lane) * 8u : kNoLoad;
  auto gload = [&](int st) {
    Stage2 r;
    r.a = stage_chunk(a.q, a.dout, g.z + st * kStageTok + tok, a.total_q, H, head, hs, lane);
    r.b = bload(rx, lane < 8 ? aux0 + (uint32_t)st * (kStageTok * 8u) : aux0);
    return r;
  };
  auto lstore = [&](int buf, const Stage2& r) {
    put_half<kHalfRows>(lane < 32 ? sQ[buf] : sDO[buf], tok, hs, r.a);
    if (lane < 8) {
      const int q = 16 * wave + 2 * lane;
      *reinterpret_cast<float2*>(&sLse[buf][q]) = make_float2(__int_as_float(r.b.x), __int_as_float(r.b.z));
      *reinterpret_cast<float2*>(&sDel[buf][q]) = make_float2(__int_as_float(r.b.y), __int_as_float(r.b.w));
    }
  };

  f32x4 dva[T][2], dka[T][2];
#pragma unroll
  for (int u = 0; u < T; ++u) dva[u][0] = dva[u][1] = dka[u][0] = dka[u][1] = f32x4{};
  // One query tile of the staged pair: every block's score and dP MFMAs,
  // then each key block's exponentials, dV and dK.
  struct Ops { bf16x8 qa[2], dot, qt; bf16x4 da[2]; f32x4 ls[2], dl[2]; };
  auto ops = [&](int buf, int j) {
    Ops o;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      o.qa[qb] = half_row8<kHalfRows>(sQ[buf], 32 * j + 16 * qb + c16, grp & 1);
      o.da[qb] = half_row4<kHalfRows>(sDO[buf], 32 * j + 16 * qb + c16, grp);
      o.ls[qb] = ldsf4(&sLse[buf][32 * j + 16 * qb + 4 * grp]);
      o.dl[qb] = ldsf4(&sDel[buf][32 * j + 16 * qb + 4 * grp]);
    }
    o.dot = tr_operand<kHalfRows>(sDO[buf], 32 * j, c16, grp);
    o.qt = tr_operand<kHalfRows>(sQ[buf], 32 * j, c16, grp);
    return o;
  };
  auto tile = [&](const Ops& o, int q0) {
    const bf16x8* qa = o.qa;
    const bf16x4* da = o.da;
    const f32x4* ls = o.ls;
    const f32x4* dl = o.dl;
    const bf16x8& dot = o.dot;
    const bf16x8& qt = o.qt;
    f32x4 s[T][2][2], dp[T][2][2];   // [u][key block][query block]
#pragma unroll
    for (int u = 0; u < T; ++u)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          s[u][kb][qb] = mfma16k32(qa[qb], ks[u][kb], ls[qb]);
          dp[u][kb][qb] = mfma16k16(da[qb], vb[u][kb], dl[qb]);
        }
    if (q0 + kTile > g.w) {   // the segment's last, partial query tile
#pragma unroll
      for (int u = 0; u < T; ++u)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              s[u][kb][qb][e] = q0 + 16 * qb + 4 * grp + e < g.w ? s[u][kb][qb][e] : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < T; ++u) {
      if (u > 0 && !active[u]) continue;   // wave-uniform
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        f32x4 p[2], ds[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            p[qb][e] = fast_exp2(s[u][kb][qb][e]);
            ds[qb][e] = p[qb][e] * dp[u][kb][qb][e];
          }
        dva[u][kb] = mfma16k32(dot, cvt4x2(p[0], p[1]), dva[u][kb]);
        dka[u][kb] = mfma16k32(qt, cvt4x2(ds[0], ds[1]), dka[u][kb]);
      }
    }
  };
  stage_walk(n_stages, gload, lstore, [&](int buf, int st) {
    if (!active[0]) return;
    stage_tiles(buf, st, n_tiles, ops, tile, g.z + st * kStageTok);
  });
#pragma unroll
  for (int u = 0; u < T; ++u)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int t = o0 + u * kTile + 16 * kb + c16;
      if (t >= g.y) continue;
      store_dims4(a.dv + ((size_t)t * H + head) * kHd, dva[u][kb], 1.f, grp);
      store_dims4(a.dk + ((size_t)t * H + head) * kHd, dka[u][kb], a.scale, grp);
    }
}

// ------------------------------------------------------------------ prep

struct DensePrep {
  const int* cu_q; const int* cu_k; int nseg;
  int total_q, total_k, heads, tq_pad, tk_tiles;
  int4* plan_q; int* count_q; int4* plan_k; int* count_k;
  int gtok_q, gtok_k;                                 // tokens per group of each plan
  const bf16* k; float* knorm;                       // forward
  float2* aux;                                       // backward: padding rows of the row statistics
  int nb_plan_k, nb_knorm, nb_rows;
};

// Row statistics of the dK/dV pass: aux.x = -LSE2 (LSE2 = log2(e) LSE;
// -1e30 for rows without keys and padding, so their P is 0), aux.y = -D =
// -rowsum(dO * O).  The dQ kernel writes them for every query of a segment as
// it computes its own seeds; this pass writes the rows after the last
// segment, [cu_q[nseg], tq_pad): the padding up to the 32-row boundary and
// any rows of q that no segment covers (cu_q[nseg] < total_q), which dK/dV's
// last partial tile stages (masked, but its dS = P dP must stay finite).
// Block-strided over (row, head), head fastest.
DEVI void dense_rows_block(const DensePrep& p, int b, int tid) {
  const int t0 = min(max(p.cu_q[p.nseg], 0), p.total_q);
  const long n = (long)p.heads * (p.tq_pad - t0);
  for (long idx = (long)b * 256 + tid; idx < n; idx += (long)p.nb_rows * 256) {
    const int h = (int)(idx % p.heads), t = t0 + (int)(idx / p.heads);
    p.aux[(size_t)h * p.tq_pad + t] = make_float2(kDeadRow, -0.f);
  }
}

__global__ __launch_bounds__(256) void dense_prep_kernel(const DensePrep p) {
  const int tid = threadIdx.x;
  int b = blockIdx.x;
  if (b == 0) { seg_plan_block(p.cu_q, p.cu_k, p.nseg, p.gtok_q, p.plan_q, p.count_q, tid); return; }
  b -= 1;
  if (b < p.nb_plan_k) { seg_plan_block(p.cu_k, p.cu_q, p.nseg, p.gtok_k, p.plan_k, p.count_k, tid); return; }
  b -= p.nb_plan_k;
  if (b < p.nb_knorm) { knorm_block(p.k, p.total_k, p.heads, p.tk_tiles, p.knorm, b, tid); return; }
  b -= p.nb_knorm;
  if (b < p.nb_rows) dense_rows_block(p, b, tid);
}

// ------------------------------------------------------------------ host side

size_t al256(size_t x) { return (x + 255) & ~size_t(255); }
int r32(int x) { return (x + kTile - 1) / kTile * kTile; }

// Groups of one direction: at most ceil(T / group) + (number of non-empty
// segments) <= ceil(T / 128) + T for any group of at least 128 tokens.
size_t plan_bytes(int total) { return al256(((size_t)(total + kGroupTok - 1) / kGroupTok + (size_t)total + 1) * 16); }

struct DenseWs { size_t counts, plan_q, plan_k, knorm, aux, total; };

DenseWs dense_ws(int total_q, int total_k, int heads, bool backward) {
  DenseWs w{};
  size_t off = 0;
  w.counts = off; off += 256;
  w.plan_q = off; off += plan_bytes(total_q);
  if (backward) {
    w.plan_k = off; off += plan_bytes(total_k);
    w.aux = off; off += al256((size_t)heads * r32(total_q) * 8);
  } else {
    w.knorm = off; off += al256((size_t)heads * (r32(total_k) / kTile) * 4);
  }
  w.total = off;
  return w;
}

unsigned group_grid(int total_outer, int nseg, int heads, int gtok) {
  return group_blocks((total_outer + gtok - 1) / gtok + min(nseg, total_outer), heads);
}

}  // namespace

int dense_attn_workspace_size(int total_q, int total_k, int heads, int head_dim, bool backward, size_t* bytes) {
  if (head_dim == kHd) {   // either kernel set (dropout runs the wide kernels)
    *bytes = max(dense_ws(total_q, total_k, heads, backward).total,
                 wide_attn_workspace_size(total_q, total_k, heads, head_dim, backward));
    return ESA_OK;
  }
  if (head_dim != 24 && head_dim != 32 && head_dim != 64) return ESA_ERR_HEAD_DIM;
  *bytes = wide_attn_workspace_size(total_q, total_k, heads, head_dim, backward);
  return ESA_OK;
}

int dense_attn_fwd(const DenseAttnCall& c, void* workspace, size_t workspace_bytes, hipStream_t st) {
  if (c.head_dim != kHd || c.dropout) return wide_attn_fwd(c, workspace, workspace_bytes, st);
  const DenseWs w = dense_ws(c.total_q, c.total_k, c.heads, false);
  if (workspace_bytes < w.total) return ESA_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  DensePrep p{};
  p.cu_q = c.cu_q; p.cu_k = c.cu_k; p.nseg = c.nseg;
  p.total_q = c.total_q; p.total_k = c.total_k; p.heads = c.heads;
  p.tq_pad = r32(c.total_q); p.tk_tiles = r32(c.total_k) / kTile;
  p.count_q = reinterpret_cast<int*>(ws + w.counts);
  p.plan_q = reinterpret_cast<int4*>(ws + w.plan_q);
  p.k = static_cast<const bf16*>(c.k); p.knorm = reinterpret_cast<float*>(ws + w.knorm);
  p.gtok_q = kFwdGroup;
  p.nb_plan_k = 0; p.nb_knorm = p.tk_tiles; p.nb_rows = 0;
  ESA_TIMED(esa_profile::kAttnPrep, st,
            hipLaunchKernelGGL(dense_prep_kernel, dim3(1 + p.nb_knorm), dim3(256), 0, st, p));
  ESA_LAUNCH_CHECK();
  DenseArgs a{};
  a.q = static_cast<const bf16*>(c.q); a.k = static_cast<const bf16*>(c.k); a.v = static_cast<const bf16*>(c.v);
  a.knorm = p.knorm; a.tk_tiles = p.tk_tiles;
  a.groups = p.plan_q; a.count = p.count_q;
  a.total_q = c.total_q; a.total_k = c.total_k; a.heads = c.heads; a.tq_pad = p.tq_pad;
  a.scale = c.scale; a.c = c.scale * kLog2e;
  a.o = static_cast<bf16*>(c.out); a.lse_out = c.lse;
  ESA_TIMED(esa_profile::kAttnFwd, st,
            hipLaunchKernelGGL(dense_fwd_kernel, dim3(group_grid(c.total_q, c.nseg, c.heads, kFwdGroup)), dim3(256), 0,
                               st, a));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

int dense_attn_bwd(const DenseAttnCall& c, void* workspace, size_t workspace_bytes, hipStream_t st) {
  if (c.head_dim != kHd || c.dropout) return wide_attn_bwd(c, workspace, workspace_bytes, st);
  const DenseWs w = dense_ws(c.total_q, c.total_k, c.heads, true);
  if (workspace_bytes < w.total) return ESA_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  DensePrep p{};
  p.cu_q = c.cu_q; p.cu_k = c.cu_k; p.nseg = c.nseg;
  p.total_q = c.total_q; p.total_k = c.total_k; p.heads = c.heads;
  p.tq_pad = r32(c.total_q); p.tk_tiles = r32(c.total_k) / kTile;
  p.count_q = reinterpret_cast<int*>(ws + w.counts);
  p.count_k = p.count_q + 1;
  p.plan_q = reinterpret_cast<int4*>(ws + w.plan_q);
  p.plan_k = reinterpret_cast<int4*>(ws + w.plan_k);
  p.aux = reinterpret_cast<float2*>(ws + w.aux);
  p.gtok_q = kDqGroup; p.gtok_k = kDkdvGroup;
  p.nb_plan_k = 1; p.nb_knorm = 0; p.nb_rows = (int)max(1L, ((long)c.heads * (p.tq_pad - c.total_q) + 255) / 256);
  ESA_TIMED(esa_profile::kAttnPrep, st,
            hipLaunchKernelGGL(dense_prep_kernel, dim3(2 + p.nb_rows), dim3(256), 0, st, p));
  ESA_LAUNCH_CHECK();
  DenseArgs a{};
  a.q = static_cast<const bf16*>(c.q); a.k = static_cast<const bf16*>(c.k); a.v = static_cast<const bf16*>(c.v);
  a.out = static_cast<const bf16*>(c.out_in); a.dout = static_cast<const bf16*>(c.dout);
  a.lse = c.lse_in; a.aux = p.aux; a.aux_out = p.aux;
  a.total_q = c.total_q; a.total_k = c.total_k; a.heads = c.heads; a.tq_pad = p.tq_pad;
  a.scale = c.scale; a.c = c.scale * kLog2e;
  a.dq = static_cast<bf16*>(c.dq); a.dk = static_cast<bf16*>(c.dk); a.dv = static_cast<bf16*>(c.dv);
  // dQ first: it writes the row statistics that dK/dV stages
  a.groups = p.plan_q; a.count = p.count_q;
  ESA_TIMED(esa_profile::kAttnBwdDq, st,
            hipLaunchKernelGGL(dense_dq_kernel, dim3(group_grid(c.total_q, c.nseg, c.heads, kDqGroup)), dim3(256), 0,
                               st, a));
  ESA_LAUNCH_CHECK();
  a.groups = p.plan_k; a.count = p.count_k;
  ESA_TIMED(esa_profile::kAttnBwdDkdv, st,
            hipLaunchKernelGGL(dense_dkdv_kernel, dim3(group_grid(c.total_k, c.nseg, c.heads, kDkdvGroup)), dim3(256),
                               0, st, a));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}
