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
constexpr int kPlanBuckets = 1024;

// Build-time tuning: issue both tiles' score MFMAs of a stage before either
// tile's exponentials (1), or finish one tile before starting the next (0);
// minimum waves per SIMD each kernel is compiled for (0 = compiler's choice).
#ifndef ESA_DENSE_PAIRED
#define ESA_DENSE_PAIRED 0
#endif
#ifndef ESA_DENSE_WAVES_FWD
#define ESA_DENSE_WAVES_FWD 0
#endif
#ifndef ESA_DENSE_WAVES_DQ
#define ESA_DENSE_WAVES_DQ 0
#endif
#ifndef ESA_DENSE_WAVES_DKDV
#define ESA_DENSE_WAVES_DKDV 0
#endif
#define ESA_WAVES_ATTR(n) __attribute__((amdgpu_waves_per_eu(n > 0 ? n : 1)))

struct DenseArgs {
  const bf16* q; const bf16* k; const bf16* v; const bf16* out; const bf16* dout;
  const uint2* aux;            // dK/dV: per (head, query) bf16 (hi, lo) pairs of -LSE2 and of -D, [H][tq_pad]
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
// consecutive heads, so with 16 heads the blocks are mapped so that XCD x
// serves the heads of one line (4 (x / 2) .. 4 (x / 2) + 3) and every other
// group (parity x % 2): each line is fetched by two XCDs, not four.  Other
// head counts use head = b % heads.
#ifndef ESA_DENSE_XCD_LINES
#define ESA_DENSE_XCD_LINES 1
#endif

DEVI void block_item_head(int H, int& item, int& head) {
  const int b = blockIdx.x;
  if (ESA_DENSE_XCD_LINES && H == 16) {
    const int xcd = b & 7, slot = b >> 3;
    head = 4 * (xcd >> 1) + (slot & 3);
    item = 2 * (slot >> 2) + (xcd & 1);
  } else {
    item = b / H;
    head = b - item * H;
  }
}

unsigned group_blocks(int groups, int H) {
  if (ESA_DENSE_XCD_LINES && H == 16) return (unsigned)(((groups + 1) / 2) * 2 * H);
  return (unsigned)(groups * H);
}

// ------------------------------------------------------------------ staging

// The stage token this lane stages (wave w: tokens 16w .. 16w+15) and its half.
DEVI int stage_tok(int wave, int lane) { return 16 * wave + ((lane & 31) >> 1); }

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

// LDS writes of one staged 16-byte chunk (8 dims of token `tok` of the stage).
DEVI void put_row(bf16* rows, int tok, int hf, i32x4 v) {
  *reinterpret_cast<i32x4*>(&rows[tok * kRowStride + 8 * hf]) = v;
}
template <int ROWS>   // tr2: two [ROWS][kTrStride] tiles (rows 0..15: the dims)
DEVI void put_col(bf16* tr2, int tok, int hf, i32x4 v) {
  const bf16x8 x = as_bf16x8(v);
  bf16* t = tr2 + (tok >> 5) * (ROWS * kTrStride) + (tok & 31);
#pragma unroll
  for (int e = 0; e < 8; ++e) t[(8 * hf + e) * kTrStride] = x[e];
}

// Loads of stage `st` issued two stages ahead, two LDS buffers, one barrier
// per stage.  gload(st) returns this lane's staging registers, lstore(buf, r)
// writes them, compute(buf, st) consumes a staged stage.  Past the end the
// loads re-read the last stage and are never stored; the loop is unrolled
// by two so the staging registers never move.
template <class Load, class Store, class Compute>
DEVI void stage_walk(int n_stages, Load gload, Store lstore, Compute compute) {
  if (n_stages <= 0) return;
  auto ra = gload(0);
  auto rb = gload(min(1, n_stages - 1));
  lstore(0, ra);
  __syncthreads();
  for (int st = 0; st < n_stages; st += 2) {
    ra = gload(min(st + 2, n_stages - 1));
    compute(0, st);
    if (st + 1 < n_stages) lstore(1, rb);
    __syncthreads();
    if (st + 1 >= n_stages) break;
    rb = gload(min(st + 3, n_stages - 1));
    compute(1, st + 1);
    if (st + 2 < n_stages) lstore(0, ra);
    __syncthreads();
  }
}

struct Stage2 { i32x4 a, b; };

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
  __shared__ __align__(16) bf16 sK[2][kStageTok * kRowStride];   // K rows [key][16]
  __shared__ __align__(16) bf16 sVT[2][2][32 * kTrStride];        // per tile [V^T ; 1]: rows 0..15 dims, 16..31 ones
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5, hf = lane & 1;
  const int H = a.heads;
  int item, head;
  block_item_head(H, item, head);
  if (item >= *a.count) return;
  const int4 g = a.groups[item];

  for (int i = tid; i < 2 * 2 * 16 * kTrStride; i += 256) {
    const int tile = i / (16 * kTrStride);
    sVT[tile >> 1][tile & 1][16 * kTrStride + (i - tile * 16 * kTrStride)] = (bf16)1.f;
  }
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
  const int tok = stage_tok(wave, lane);
  auto gload = [&](int st) { return stage_chunk(a.k, a.v, g.z + st * kStageTok + tok, a.total_k, H, head, hf, lane); };
  auto lstore = [&](int buf, i32x4 r) {
    if (lane < 32) put_row(sK[buf], tok, hf, r);
    else put_col<32>(&sVT[buf][0][0], tok, hf, r);
  };

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
    auto k_rows = [&](int buf, int j) { return lds8(&sK[buf][(32 * j + kperm(col)) * kRowStride + 8 * half]); };
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
    // One key tile of the staged pair: the score MFMAs of all query tiles
    // first, then each query tile's softmax and P V.
    auto tile = [&](int buf, int j, int k0) {
      const bf16x8 kr = k_rows(buf, j);
      f32x16 s[T];
#pragma unroll
      for (int u = 0; u < T; ++u) s[u] = scores(kr, u);
      const bf16x8 vt0 = lds8(&sVT[buf][j][col * kTrStride + 8 * half]);
      const bf16x8 vt1 = lds8(&sVT[buf][j][col * kTrStride + 16 + 8 * half]);
#pragma unroll
      for (int u = 0; u < T; ++u)
        if (u == 0 || active[u]) softmax_pv(u, s[u], k0, vt0, vt1);   // active[u]: wave-uniform
    };
    stage_walk(n_stages, gload, lstore, [&](int buf, int st) {
      if (!any_active) return;
      const int k0 = g.z + st * kStageTok;
      tile(buf, 0, k0);
      if (2 * st + 1 < n_tiles) tile(buf, 1, k0 + kTile);
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
// One wave = 32 queries (lanes); dQ = scale * sum_k P (dP - D) k with
// S' = K (c q)^T - LSE2 from two MFMAs seeded with -LSE2, P = exp2(S').

__global__ __launch_bounds__(256) ESA_WAVES_ATTR(ESA_DENSE_WAVES_DQ) void dense_dq_kernel(const DenseArgs a) {
  __shared__ __align__(16) bf16 sK[2][kStageTok * kRowStride];    // K rows
  __shared__ __align__(16) bf16 sV[2][kStageTok * kRowStride];    // V rows
  __shared__ __align__(16) bf16 sKT[2][2][16 * kTrStride];         // K^T per tile
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5, hf = lane & 1;
  const int H = a.heads;
  int item, head;
  block_item_head(H, item, head);
  if (item >= *a.count) return;
  const int4 g = a.groups[item];

  const int o0 = g.x + wave * kTile;
  const bool active = o0 < g.y;
  const int t = o0 + col;
  const bool valid = t < g.y;
  const int tc = valid ? t : g.x;
  const size_t row = ((size_t)tc * H + head) * kHd + 8 * half;
  const bf16x8 qf = *reinterpret_cast<const bf16x8*>(a.q + row);
  const bf16x8 dof = *reinterpret_cast<const bf16x8*>(a.dout + row);
  const bf16x8 of = *reinterpret_cast<const bf16x8*>(a.out + row);
  float dsum = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) dsum = fmaf((float)dof[e], (float)of[e], dsum);
  dsum += __shfl_xor(dsum, 32);
  const float lq = a.lse[(size_t)head * a.total_q + tc];
  const f32x16 cl = splat16(lq == -INFINITY ? -INFINITY : -lq * kLog2e);   // seed of S': -LSE2
  const f32x16 cd = splat16(-dsum);                                        // seed of dP: -D
  bf16x8 qh, ql;
  split_scaled(qf, a.c, qh, ql);

  const int n_tiles = (g.w - g.z + kTile - 1) >> 5;
  const int n_stages = (n_tiles + 1) >> 1;
  const int tok = stage_tok(wave, lane);
  auto gload = [&](int st) { return stage_chunk(a.k, a.v, g.z + st * kStageTok + tok, a.total_k, H, head, hf, lane); };
  auto lstore = [&](int buf, i32x4 r) {
    if (lane < 32) {
      put_row(sK[buf], tok, hf, r);
      put_col<16>(&sKT[buf][0][0], tok, hf, r);
    } else {
      put_row(sV[buf], tok, hf, r);
    }
  };

  f32x16 acc = {};
  struct SP { f32x16 s, dp; };
  auto scores = [&](int buf, int j) {
    const int rrow = (32 * j + kperm(col)) * kRowStride + 8 * half;
    const bf16x8 kr = lds8(&sK[buf][rrow]);
    return SP{mfma32(kr, ql, mfma32(kr, qh, cl)), mfma32(lds8(&sV[buf][rrow]), dof, cd)};
  };
  auto tile = [&](int buf, int j, int k0, SP sp) {
    f32x16& s = sp.s;
    const f32x16& dp = sp.dp;
    if (k0 + kTile > g.w) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = k0 + row_local(r, half) < g.w ? s[r] : -INFINITY;
    }
    float ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) ds[r] = fast_exp2(s[r]) * dp[r];
    const int trow = (col & 15) * kTrStride + 8 * half;
    acc = mfma32(lds8(&sKT[buf][j][trow]), cvt8(ds), acc);
    acc = mfma32(lds8(&sKT[buf][j][trow + 16]), cvt8(ds + 8), acc);
  };
  stage_walk(n_stages, gload, lstore, [&](int buf, int st) {
    if (!active) return;
    const int k0 = g.z + st * kStageTok;
    if (ESA_DENSE_PAIRED && 2 * st + 1 < n_tiles) {
      const SP s0 = scores(buf, 0), s1 = scores(buf, 1);
      tile(buf, 0, k0, s0);
      tile(buf, 1, k0 + kTile, s1);
    } else {
      tile(buf, 0, k0, scores(buf, 0));
      if (2 * st + 1 < n_tiles) tile(buf, 1, k0 + kTile, scores(buf, 1));
    }
  });
  if (!valid) return;
  store_rows8(a.dq + ((size_t)t * H + head) * kHd, acc, a.scale, half);
}

// ------------------------------------------------------------------ dK/dV pass
// One wave = 32 keys (lanes); rows are queries.  S' = Q (c k)^T - LSE2 with
// -LSE2 broadcast per row by an MFMA of its bf16 (hi, lo) halves against a
// ones column, likewise dP' = dO v^T - D; dV = P^T dO, dK = scale dS^T Q.
// A query's statistics sit in one 16-byte LDS record {-LSE2 pair, -D pair,
// 0, 0}: read once, it is the A operand of both statistic MFMAs, whose B
// operands select the pair (ones in k slots 0, 1 or 2, 3).

__global__ __launch_bounds__(256) ESA_WAVES_ATTR(ESA_DENSE_WAVES_DKDV) void dense_dkdv_kernel(const DenseArgs a) {
  __shared__ __align__(16) bf16 sQ[2][kStageTok * kRowStride];
  __shared__ __align__(16) bf16 sDO[2][kStageTok * kRowStride];
  __shared__ __align__(16) bf16 sQT[2][2][16 * kTrStride];
  __shared__ __align__(16) bf16 sDOT[2][2][16 * kTrStride];
  __shared__ __align__(16) i32x4 sAux[2][kStageTok];   // per query {-LSE2 pair, -D pair, 0, 0}
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5, hf = lane & 1;
  const int H = a.heads;
  int item, head;
  block_item_head(H, item, head);
  if (item >= *a.count) return;
  const int4 g = a.groups[item];   // outer = keys, inner = queries

  const int o0 = g.x + wave * kTile;
  const bool active = o0 < g.y;
  const int t = o0 + col;
  const bool valid = t < g.y;
  const int tc = valid ? t : g.x;
  const size_t row = ((size_t)tc * H + head) * kHd + 8 * half;
  const bf16x8 kf = *reinterpret_cast<const bf16x8*>(a.k + row);
  const bf16x8 vf = *reinterpret_cast<const bf16x8*>(a.v + row);
  bf16x8 kh, kl;
  split_scaled(kf, a.c, kh, kl);
  // B operands of the row-statistic MFMAs: ones in k slots 0, 1 (the -LSE2
  // pair of the record) or 2, 3 (the -D pair); half-1 lanes carry k 8..15.
  bf16x8 ones_s = {}, ones_d = {};
  if (half == 0) {
    ones_s[0] = ones_s[1] = (bf16)1.f;
    ones_d[2] = ones_d[3] = (bf16)1.f;
  }

  const int n_tiles = (g.w - g.z + kTile - 1) >> 5;
  const int n_stages = (n_tiles + 1) >> 1;
  const rsrc_t rx = make_rsrc(a.aux + (size_t)head * a.tq_pad, (uint32_t)a.tq_pad * 8u);
  const int tok = stage_tok(wave, lane);
  // row statistics: lanes 0..7 of wave w fetch queries 16w .. 16w+15 (two 8-byte records per lane)
  const uint32_t aux0 = lane < 8 ? (uint32_t)(g.z + 16 * wave + 2 * lane) * 8u : kNoLoad;
  auto gload = [&](int st) {
    Stage2 r;
    r.a = stage_chunk(a.q, a.dout, g.z + st * kStageTok + tok, a.total_q, H, head, hf, lane);
    r.b = bload(rx, lane < 8 ? aux0 + (uint32_t)st * (kStageTok * 8u) : aux0);
    return r;
  };
  auto lstore = [&](int buf, const Stage2& r) {
    if (lane < 32) {
      put_row(sQ[buf], tok, hf, r.a);
      put_col<16>(&sQT[buf][0][0], tok, hf, r.a);
    } else {
      put_row(sDO[buf], tok, hf, r.a);
      put_col<16>(&sDOT[buf][0][0], tok, hf, r.a);
    }
    if (lane < 8) {
      sAux[buf][16 * wave + 2 * lane] = i32x4{r.b.x, r.b.y, 0, 0};
      sAux[buf][16 * wave + 2 * lane + 1] = i32x4{r.b.z, r.b.w, 0, 0};
    }
  };

  f32x16 dva = {}, dka = {};
  const f32x16 zero = {};
  struct SP { f32x16 s, dp; };
  auto scores = [&](int buf, int j) {
    const int rrow = (32 * j + kperm(col)) * kRowStride + 8 * half;
    const bf16x8 ax = as_bf16x8(sAux[buf][32 * j + kperm(col)]);
    const bf16x8 qr = lds8(&sQ[buf][rrow]);
    return SP{mfma32(qr, kl, mfma32(qr, kh, mfma32(ax, ones_s, zero))),
              mfma32(lds8(&sDO[buf][rrow]), vf, mfma32(ax, ones_d, zero))};
  };
  auto tile = [&](int buf, int j, int q0, const SP& sp) {
    const f32x16& s = sp.s;
    const f32x16& dp = sp.dp;
    float p[16], ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = fast_exp2(s[r]);
    if (q0 + kTile > g.w) {
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = q0 + row_local(r, half) < g.w ? p[r] : 0.f;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) ds[r] = p[r] * dp[r];
    const int trow = (col & 15) * kTrStride + 8 * half;
    dva = mfma32(lds8(&sDOT[buf][j][trow]), cvt8(p), dva);
    dva = mfma32(lds8(&sDOT[buf][j][trow + 16]), cvt8(p + 8), dva);
    dka = mfma32(lds8(&sQT[buf][j][trow]), cvt8(ds), dka);
    dka = mfma32(lds8(&sQT[buf][j][trow + 16]), cvt8(ds + 8), dka);
  };
  stage_walk(n_stages, gload, lstore, [&](int buf, int st) {
    if (!active) return;
    const int q0 = g.z + st * kStageTok;
    if (ESA_DENSE_PAIRED && 2 * st + 1 < n_tiles) {
      const SP s0 = scores(buf, 0), s1 = scores(buf, 1);
      tile(buf, 0, q0, s0);
      tile(buf, 1, q0 + kTile, s1);
    } else {
      tile(buf, 0, q0, scores(buf, 0));
      if (2 * st + 1 < n_tiles) tile(buf, 1, q0 + kTile, scores(buf, 1));
    }
  });
  if (!valid) return;
  store_rows8(a.dv + ((size_t)t * H + head) * kHd, dva, 1.f, half);
  store_rows8(a.dk + ((size_t)t * H + head) * kHd, dka, a.scale, half);
}

// ------------------------------------------------------------------ prep

// Groups of one direction: every segment's outer tokens cut into groups of
// `gtok` tokens (one block each), segments ordered by partner tiles (longest first, counting sort in
// one block; segments with equal counts in any order, which changes no
// result).  groups[i] = (outer begin, outer segment end, inner begin, inner end).
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

struct DensePrep {
  const int* cu_q; const int* cu_k; int nseg;
  int total_q, total_k, heads, tq_pad, tk_tiles;
  int4* plan_q; int* count_q; int4* plan_k; int* count_k;
  int gtok_q, gtok_k;                                 // tokens per group of each plan
  const bf16* k; float* knorm;                       // forward
  const bf16* out; const bf16* dout; const float* lse; uint2* aux;   // backward
  int nb_plan_k, nb_knorm, nb_rows;
};

// Row statistics of the dK/dV pass as bf16 (hi, lo) pairs: aux.x = -LSE2
// (LSE2 = log2(e) LSE; -1e30 for rows without keys and padding, so their P is
// 0), aux.y = -D = -rowsum(dO * O).  Thread per (query, head), head fastest.
DEVI void dense_rows_item(const DensePrep& p, long idx) {
  if (idx >= (long)p.heads * p.tq_pad) return;
  const int h = (int)(idx % p.heads), t = (int)(idx / p.heads);
  float xs = kDeadRow, dsum = 0.f;
  if (t < p.total_q) {
    const float l = p.lse[(size_t)h * p.total_q + t];
    if (l != -INFINITY) xs = -(l * kLog2e);
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

__global__ __launch_bounds__(256) void dense_prep_kernel(const DensePrep p) {
  const int tid = threadIdx.x;
  int b = blockIdx.x;
  if (b == 0) { seg_plan_block(p.cu_q, p.cu_k, p.nseg, p.gtok_q, p.plan_q, p.count_q, tid); return; }
  b -= 1;
  if (b < p.nb_plan_k) { seg_plan_block(p.cu_k, p.cu_q, p.nseg, p.gtok_k, p.plan_k, p.count_k, tid); return; }
  b -= p.nb_plan_k;
  if (b < p.nb_knorm) { knorm_block(p.k, p.total_k, p.heads, p.tk_tiles, p.knorm, b, tid); return; }
  b -= p.nb_knorm;
  if (b < p.nb_rows) dense_rows_item(p, (long)b * 256 + tid);
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

size_t dense_attn_workspace_size(int total_q, int total_k, int heads, bool backward) {
  return dense_ws(total_q, total_k, heads, backward).total;
}

int dense_attn_fwd(const DenseAttnCall& c, void* workspace, size_t workspace_bytes, hipStream_t st) {
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
  p.out = static_cast<const bf16*>(c.out_in); p.dout = static_cast<const bf16*>(c.dout); p.lse = c.lse_in;
  p.aux = reinterpret_cast<uint2*>(ws + w.aux);
  p.gtok_q = kGroupTok; p.gtok_k = kGroupTok;
  p.nb_plan_k = 1; p.nb_knorm = 0; p.nb_rows = (int)(((long)c.heads * p.tq_pad + 255) / 256);
  ESA_TIMED(esa_profile::kAttnPrep, st,
            hipLaunchKernelGGL(dense_prep_kernel, dim3(2 + p.nb_rows), dim3(256), 0, st, p));
  ESA_LAUNCH_CHECK();
  DenseArgs a{};
  a.q = static_cast<const bf16*>(c.q); a.k = static_cast<const bf16*>(c.k); a.v = static_cast<const bf16*>(c.v);
  a.out = static_cast<const bf16*>(c.out_in); a.dout = static_cast<const bf16*>(c.dout);
  a.lse = c.lse_in; a.aux = p.aux;
  a.total_q = c.total_q; a.total_k = c.total_k; a.heads = c.heads; a.tq_pad = p.tq_pad;
  a.scale = c.scale; a.c = c.scale * kLog2e;
  a.dq = static_cast<bf16*>(c.dq); a.dk = static_cast<bf16*>(c.dk); a.dv = static_cast<bf16*>(c.dv);
  a.groups = p.plan_k; a.count = p.count_k;
  ESA_TIMED(esa_profile::kAttnBwdDkdv, st,
            hipLaunchKernelGGL(dense_dkdv_kernel, dim3(group_grid(c.total_k, c.nseg, c.heads, kGroupTok)), dim3(256),
                               0, st, a));
  ESA_LAUNCH_CHECK();
  a.groups = p.plan_q; a.count = p.count_q;
  ESA_TIMED(esa_profile::kAttnBwdDq, st,
            hipLaunchKernelGGL(dense_dq_kernel, dim3(group_grid(c.total_q, c.nseg, c.heads, kGroupTok)), dim3(256), 0,
                               st, a));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}
