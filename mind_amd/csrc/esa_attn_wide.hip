// Dense varlen attention (no mask) at head dims 24, 32 and 64, bf16 operands,
// fp32 softmax, on gfx950: the flash_attn_varlen_func drop-in
// (esa/mha_flash_varlen.py:177-184, causal=False) for the ESA configurations
// whose dim / num_heads is 24, 32 or 64 (esa/mha.py:50-52), and, with
// attention dropout (DROP), for every head dim including 16.  Products over
// partners compute 32 output dims per block: head dims 16 and 24 read their
// rows as two / three 8-dim octets, the other octets of every operand are
// zero, and output dims past the head dim are not stored.
//
// Dropout: the keep mask of esa_common.h, from each lane's own row (forward,
// dQ) or column (dK/dV) key and the staged partners' keys, computed once per
// token during staging and held in LDS beside the rows; a dropped partner's
// probability is zeroed in the products over partners (and its dP in dS),
// the outputs carry 1 / (1 - p), the softmax statistics are undropped.
//
// Work items are 128-token groups cut from each segment on its own (the
// segment plans of the head-dim-16 kernels): a block's four waves own four
// consecutive 32-token tiles of one segment and one head and walk the same
// partner range, staged 64 tokens at a time into double-buffered LDS (one
// barrier per stage, the next stage's global loads in flight in registers).
//
// Register layouts (v_mfma_f32_32x32x16_bf16, helpers in esa_attn_tiles.h):
//  - Scores: S^T = X Y^T summed over head_dim / 16 chunks of 16 dims, the
//    partner rows X in the A operand from LDS with rows permuted (kperm), the
//    owned token's row in the B operand from registers.  Lane l owns token
//    column l % 32; its 16 accumulators hold partners row_local(r, l / 32):
//    registers 0..7 are partners 8 h .. 8 h + 7 and 8..15 are 16 + 8 h ..,
//    exactly the K slots lane l supplies to a product over the tile's
//    partners (h = l / 32), so probabilities feed the next MFMA's B operand
//    without data movement.
//  - Products over partners (P V, dS K, P^T dO, dS^T Q): M = 32 output dims
//    per block (head_dim / 32 blocks), the A operand [dims x partners] from
//    LDS transpose reads (ds_read_b64_tr_b16) of the staged rows.
//  - LDS rows: [dim octet][token][8 dims], octet stride padded by 4 tokens so
//    the two octets of a transpose read fall in different banks.
// The softmax scale c = scale * log2(e) is applied inside the exponent (one
// FMA per score, exp2(c s - c m)); the backward's -LSE2 / c and -D row
// statistics are MFMA accumulator seeds.  Forward reference point: by
// Cauchy-Schwarz c |s| <= c |q| max|k|; when that bound is <= 60 for all of a
// wave's queries over their partner range (max |k| per 32-key tile from the
// prep pass), exp2(c s) stays in [2^-60, 2^60] and the wave skips the running
// maximum and its rescales; otherwise the online path runs.  The row sum adds
// the bf16 probabilities the P V products take (v_dot2c_f32_bf16), so the
// normalisation matches the products exactly (a one-key row gives out = v).  Every sum has a fixed order: the
// backward is deterministic (dQ pass, then dK/dV pass; no atomics).
#include "esa_attn_tiles.h"
#include "esa_attn_dense.h"
#include "esa_profile.h"
#include "../../include/esa_hip.h"

namespace {

// Build-time tuning: minimum waves per SIMD the dK/dV kernel is compiled for
// (0 = the compiler's choice).
#ifndef ESA_WIDE_WAVES_DKDV
#define ESA_WIDE_WAVES_DKDV 0
#endif
// Minimum waves per SIMD of the dQ kernel at head dim 64.
#ifndef ESA_WIDE_WAVES_DQ64
#define ESA_WIDE_WAVES_DQ64 3
#endif
// Build-time switch: 1 = staged tokens swizzled per octet pair (below), 0 = plain layout.
#ifndef ESA_WIDE_SWZ
#define ESA_WIDE_SWZ 1
#endif

constexpr int kWStage = 64;              // partner tokens per stage (two tiles)
constexpr int kWTokPad = kWStage + 4;    // LDS octet stride in tokens

struct WideArgs {
  DropoutCfg drop;
  const float* knorm; int tk_tiles;   // forward: max |k| per (head, 32-key tile), [H][tk_tiles]
  const bf16* q; const bf16* k; const bf16* v; const bf16* out; const bf16* dout;
  const float* lse;            // dQ pass input [H][Tq]
  float2* aux;                 // per (head, query) {-LSE2 / c, -D}, [H][tq_pad]: written by dQ, read by dK/dV
  const int4* groups; const int* count;
  int total_q, total_k, heads, tq_pad;
  float c, scale;
  bf16* o; float* lse_out; bf16* dq; bf16* dk; bf16* dv;
};

// LDS position of staged token t in octet o of an NO-octet layout.  The
// octet stride (68 tokens = 1088 bytes, 64 mod 128) puts octets of equal
// parity on the same banks of a 128-byte window, where the 16-byte staging
// stores of 8 consecutive lanes (one token's 8 octets at head dim 64, two
// tokens' 4 at head dim 32) collided 4- and 2-way.  XORing the token's low
// two bits with a value per octet pair ((o / 2) mod 4 for 8 octets,
// 2 ((o / 2) mod 2) for 4) spreads them over the window's eight 16-byte
// slots.  Every read covers aligned blocks of 4 or 8 tokens of one octet
// pair, which the XOR only permutes, so the reads keep their bank pattern.
template <int NO>
DEVI int wtok(int t, int o) { return ESA_WIDE_SWZ ? t ^ (((o >> 1) & (NO / 2 - 1)) * (8 / NO)) : t; }

// 16 bytes of the A operand of a score MFMA: dims 16 c + 8 h .. + 7 (octet
// 2 c + h) of staged token t.
template <int NO>
DEVI bf16x8 row_octet(const bf16* rows, int t, int o) { return lds8(rows + ((size_t)o * kWTokPad + wtok<NO>(t, o)) * 8); }

// A operand [32 dims x 16 partners] of a product over partners: dims
// 32 m + (lane % 32), partners 16 j + 8 h .. + 7 (h = lane / 32), by two
// transpose reads of four tokens each.  In a 16-lane group, lane L
// addresses token t0 + L / 4 (+ 4 in the second read), dims 4 (L % 4) .. + 3
// of the group's 16 dims, so lane i receives dim i of the four tokens.
template <int NO>
DEVI bf16x8 tr_dims(const bf16* rows, int m, int j, int lane) {
  const int i = lane & 15, grp = lane >> 4;
  const int d = 32 * m + 16 * (grp & 1) + 4 * (i & 3);
  const int t = 16 * j + 8 * (grp >> 1) + (i >> 2), o = d >> 3;
  const bf16* p = rows + ((size_t)o * kWTokPad + wtok<NO>(t, o)) * 8 + (d & 7);
  const bf16x4 lo = lds_tr4(p), hi = lds_tr4(p + 4 * 8);
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Output dims 32 m + 8 (r / 4) + 4 h + (r % 4) of a product accumulator, 4
// consecutive dims per register quad: written as bf16 x 4.
template <int HD>
DEVI void store_acc(bf16* __restrict__ row, const f32x16 (&acc)[(HD + 31) / 32], float mul, int h) {
#pragma unroll
  for (int m = 0; m < (HD + 31) / 32; ++m)
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      if (32 * m + 8 * a >= HD) continue;   // the padding dims of head dim 24
      bf16x4 x;
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = (bf16)(acc[m][4 * a + e] * mul);
      *reinterpret_cast<bf16x4*>(row + 32 * m + 8 * a + 4 * h) = x;
    }
}

// Dims 8 o .. 8 o + 7 of a global row; zeros for the padding octet of head dim 24.
template <int HD>
DEVI bf16x8 row_op(const bf16* __restrict__ row, int o) {
  if (8 * o >= HD) return bf16x8{};
  return *reinterpret_cast<const bf16x8*>(row + 8 * o);
}

// c + the sum of the eight bf16 values of x, by v_dot2c_f32_bf16 against (1, 1).
DEVI float bf16_sum8(const bf16x8& x, float c) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 ones = {(bf16)1.f, (bf16)1.f};
#pragma unroll
  for (int i = 0; i < 4; ++i) c = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{x[2 * i], x[2 * i + 1]}, ones, c, false);
  return c;
}

// Block -> (work item, head).  Block b runs on XCD b % 8, each XCD with its
// own L2, and a 128-byte line of a [T][H][HD] bf16 tensor holds the rows of
// L = 128 / (2 HD) consecutive heads of one token (head dim 32: 2, 64: 1).
// When H is a multiple of 8 L, XCD x serves the line groups x, x + 8, ..., so
// a line's heads share one L2 and each line is fetched once (head dim 32 at 16
// heads read 1.5-2x its algorithmic bytes with head = b % H); otherwise head
// fastest, head = b % H.
template <int HD>
DEVI void wide_item_head(int H, int& item, int& head) {
  constexpr int L = HD == 32 ? 2 : 1;   // head dims 16 and 24 run only with dropout; 64 fills a line
  const int b = (int)blockIdx.x;
  if (L > 1 && H % (8 * L) == 0) {
    const int per_xcd = H / 8;   // heads served by one XCD: H / (8 L) line groups of L heads
    const int x = b & 7, slot = b >> 3;
    const int j = slot % per_xcd;
    head = (x + 8 * (j / L)) * L + j % L;
    item = slot / per_xcd;
  } else {
    item = b / H;
    head = b - item * H;
  }
}

// ---- staging: stage st covers partner tokens g0 + 64 st .. + 63 of tensors
// A and B ([T][H][HD] bf16); each thread holds CPT 16-byte chunks (token-major
// over (tensor, token, octet), so consecutive threads read consecutive bytes of
// a row) in a ring of two register sets.  The NR = HD / 8 octets of a row are
// staged; LDS holds NO = 4 ceil(HD / 32) octets per token.
template <int HD>
struct WStage {
  static constexpr int NR = HD / 8;
  static constexpr int NCH = 2 * kWStage * NR;            // chunks per stage
  static constexpr int CPT = (NCH + 255) / 256;
  i32x4 r[CPT];
};

template <int HD>
DEVI WStage<HD> wide_gload(const bf16* a, const bf16* b, int g0, int total, int H, int head, int tid) {
  constexpr int NR = HD / 8;
  WStage<HD> s;
#pragma unroll
  for (int i = 0; i < WStage<HD>::CPT; ++i) {
    const int c = tid + 256 * i;
    if (WStage<HD>::NCH % 256 != 0 && c >= WStage<HD>::NCH) { s.r[i] = i32x4{}; continue; }
    const int tensor = c / (kWStage * NR), rem = c - tensor * (kWStage * NR);
    const int tok = rem / NR, o = rem - tok * NR;
    const int t = min(g0 + tok, total - 1);
    s.r[i] = *reinterpret_cast<const i32x4*>((tensor ? b : a) + ((size_t)t * H + head) * HD + 8 * o);
  }
  return s;
}
template <int HD>
DEVI void wide_lstore(bf16* sa, bf16* sb, const WStage<HD>& s, int tid) {
  constexpr int NR = HD / 8;
#pragma unroll
  for (int i = 0; i < WStage<HD>::CPT; ++i) {
    const int c = tid + 256 * i;
    if (WStage<HD>::NCH % 256 != 0 && c >= WStage<HD>::NCH) continue;
    const int tensor = c / (kWStage * NR), rem = c - tensor * (kWStage * NR);
    const int tok = rem / NR, o = rem - tok * NR;
    *reinterpret_cast<i32x4*>((tensor ? sb : sa) + ((size_t)o * kWTokPad + wtok<(HD + 31) / 32 * 4>(tok, o)) * 8) =
        s.r[i];
  }
}
// Head dim 24: the padding octet of the four staging buffers (two tensors,
// two buffers) is zeroed once, before the first stage's barrier; staging never
// writes it.
template <int HD>
DEVI void wide_zero_pad(bf16* a0, bf16* a1, bf16* b0, bf16* b1, int tid) {
  constexpr int NR = HD / 8, NO = (HD + 31) / 32 * 4, NP = NO - NR;
  if (NP == 0) return;
  for (int i = tid; i < 4 * kWStage * NP; i += 256) {
    const int buf = i / (kWStage * NP), rem = i - buf * (kWStage * NP);
    const int tok = rem / NP, o = NR + rem - tok * NP;
    bf16* base = buf == 0 ? a0 : buf == 1 ? a1 : buf == 2 ? b0 : b1;
    *reinterpret_cast<i32x4*>(base + ((size_t)o * kWTokPad + tok) * 8) = i32x4{};
  }
}

// A stage's rows with the dropout key of partner token tid (tid < 64).
template <int HD>
struct WStageK {
  WStage<HD> rows;
  uint32_t key;
};

// Zeroes x[r] for the partners the keep mask drops: register r of lane half
// h holds partner row_local(r, h) of the tile whose 32 partner keys start at
// `keys` (LDS), the lane's own key is `own`.  Forward and dQ: the partners
// are the keys, register 8 b + e holding key base + 16 b + 8 h + e, so the
// global key pair {2i, 2i + 1} sits in two neighbouring registers of a run of
// 8 and shares one hash: with the tile base `bp` = base mod 2 even the pairs
// are registers (0, 1) .. (6, 7), 4 hashes per run; odd, (1, 2) .. (5, 6)
// with registers 0 and 7 alone (their pairs lie in other runs), 5.
DEVI void drop_tile(const DropoutCfg& d, uint32_t own, const uint32_t* keys, int h, int bp, float (&x)[16]) {
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const uint4 k0 = *reinterpret_cast<const uint4*>(keys + 16 * b + 8 * h);
    const uint4 k1 = *reinterpret_cast<const uint4*>(keys + 16 * b + 8 * h + 4);
    const uint32_t kk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
    float* y = x + 8 * b;
    if (bp == 0) {
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const uint32_t bits = drop_bits(own, kk[e]);
        y[e] = drop_half(d, bits, 0) ? y[e] : 0.f;
        y[e + 1] = drop_half(d, bits, 1) ? y[e + 1] : 0.f;
      }
    } else {
      y[0] = drop_half(d, drop_bits(own, kk[0]), 1) ? y[0] : 0.f;
#pragma unroll
      for (int e = 1; e < 7; e += 2) {
        const uint32_t bits = drop_bits(own, kk[e]);
        y[e] = drop_half(d, bits, 0) ? y[e] : 0.f;
        y[e + 1] = drop_half(d, bits, 1) ? y[e + 1] : 0.f;
      }
      y[7] = drop_half(d, drop_bits(own, kk[7]), 0) ? y[7] : 0.f;
    }
  }
}
// dK / dV (the partners are queries, the lane's own token the key, of parity
// kpar): each score takes its key's half of its own hash.
DEVI void drop_tile_key(const DropoutCfg& d, uint32_t own, const uint32_t* keys, int h, int kpar, float (&x)[16]) {
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const uint4 k0 = *reinterpret_cast<const uint4*>(keys + 16 * b + 8 * h);
    const uint4 k1 = *reinterpret_cast<const uint4*>(keys + 16 * b + 8 * h + 4);
    const uint32_t kk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) x[8 * b + e] = drop_half(d, drop_bits(kk[e], own), kpar) ? x[8 * b + e] : 0.f;
  }
}

// Two LDS buffers and two stages' loads in flight: stage s + 2 is requested
// before stage s is consumed; stage s + 1 is written to LDS after it.
template <class Load, class Store, class Compute>
DEVI void wide_walk(int n_stages, Load gload, Store lstore, Compute compute) {
  if (n_stages <= 0) return;
  auto r0 = gload(0);
  auto r1 = gload(min(1, n_stages - 1));
  lstore(0, r0);
  __syncthreads();
  for (int st = 0; st < n_stages; st += 2) {
    r0 = gload(min(st + 2, n_stages - 1));
    compute(0, st);
    if (st + 1 >= n_stages) return;
    lstore(1, r1);
    __syncthreads();
    r1 = gload(min(st + 3, n_stages - 1));
    compute(1, st + 1);
    if (st + 2 >= n_stages) return;
    lstore(0, r0);
    __syncthreads();
  }
}

constexpr int kWGroup = kWaves * kTile;   // 128 owned tokens per block

// ------------------------------------------------------------------ forward
template <int HD, bool DROP>
__global__ __launch_bounds__(256) void wide_fwd_kernel(const WideArgs a) {
  constexpr int HP = (HD + 31) / 32 * 32, NC = (HD + 15) / 16, NM = HP / 32, NO = HP / 8;
  __shared__ __align__(16) bf16 sK[2][NO * kWTokPad * 8];
  __shared__ __align__(16) bf16 sV[2][NO * kWTokPad * 8];
  __shared__ __align__(16) uint32_t sKey[2][DROP ? kWStage : 4];   // column keys of the staged keys
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, h = lane >> 5;
  const int H = a.heads;
  int item, head;
  wide_item_head<HD>(H, item, head);
  if (item >= *a.count) return;
  const int4 g = a.groups[item];
  const int t = g.x + wave * kTile + col;
  const bool valid = t < g.y, active = g.x + wave * kTile < g.y;
  const bf16* qrow = a.q + ((size_t)(valid ? t : g.x) * H + head) * HD;
  bf16x8 qop[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) qop[c] = row_op<HD>(qrow, 2 * c + h);
  wide_zero_pad<HD>(sK[0], sK[1], sV[0], sV[1], tid);
  const uint32_t rk = DROP ? drop_row(a.drop, valid ? t : g.x, head) : 0u;
  // the wave's bound c |q| max|k| over its partner range
  float km = 0.f;
  for (int tt = (g.z >> 5) + lane; tt < ((g.w + kTile - 1) >> 5); tt += 64)
    km = fmaxf(km, a.knorm[(size_t)head * a.tk_tiles + tt]);
  km = wave_max(km);
  float qq = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) qq = fmaf((float)qop[c][e], (float)qop[c][e], qq);
  qq += __shfl_xor(qq, 32);
  const float bnd = valid ? a.c * sqrtf(qq) * km : 0.f;
  const bool fixed_ref = __builtin_amdgcn_readfirstlane((int)(wave_max(bnd) <= kStaticBound)) != 0;
  f32x16 acc[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) acc[m] = f32x16{};
  float m_run = fixed_ref ? 0.f : -INFINITY, l_run = 0.f;
  const int n_tiles = (g.w - g.z + kTile - 1) >> 5;
  const int n_stages = (n_tiles + 1) >> 1;
  const f32x16 zero = {};
  auto run = [&](auto online_tag) {
  constexpr bool ONLINE = decltype(online_tag)::value;
  wide_walk(
      n_stages,
      [&](int st) {
        WStageK<HD> s;
        s.rows = wide_gload<HD>(a.k, a.v, g.z + st * kWStage, a.total_k, H, head, tid);
        s.key = DROP && tid < kWStage ? drop_col(a.drop, g.z + st * kWStage + tid) : 0u;
        return s;
      },
      [&](int buf, const WStageK<HD>& s) {
        wide_lstore<HD>(sK[buf], sV[buf], s.rows, tid);
        if (DROP && tid < kWStage) sKey[buf][tid] = s.key;
      },
      [&](int buf, int st) {
        if (!active) return;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          if (2 * st + u >= n_tiles) break;
          const int k0 = g.z + st * kWStage + u * kTile;
          f32x16 s = zero;
#pragma unroll
          for (int c = 0; c < NC; ++c) s = mfma32(row_octet<NO>(sK[buf], u * kTile + kperm(col), 2 * c + h), qop[c], s);
          if (k0 + kTile > g.w) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = k0 + row_local(r, h) < g.w ? s[r] : -INFINITY;
          }
          float p[16];
          if (ONLINE) {
            float mt = s[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float m_new = fmaxf(m_run, mt);
            if (__ballot(m_new > m_run)) {
              const float alpha = m_run == -INFINITY ? 0.f : fast_exp2(a.c * (m_run - m_new));
              l_run *= alpha;
#pragma unroll
              for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[m][r] *= alpha;
              m_run = m_new;
            }
            const float cm = m_run == -INFINITY ? 0.f : a.c * m_run;
#pragma unroll
            for (int r = 0; r < 16; ++r) p[r] = fast_exp2(fmaf(s[r], a.c, -cm));
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) p[r] = fast_exp2(s[r] * a.c);
          }
          // the row sum of exactly the bf16 probabilities the products use, two per instruction
          bf16x8 pb[2] = {cvt8(p), cvt8(p + 8)};
          l_run = bf16_sum8(pb[0], bf16_sum8(pb[1], l_run));
          if (DROP) {
            drop_tile(a.drop, rk, &sKey[buf][u * kTile], h, g.z & 1, p);
            pb[0] = cvt8(p);
            pb[1] = cvt8(p + 8);
          }
#pragma unroll
          for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[m] = mfma32(tr_dims<NO>(sV[buf], m, 2 * u + j, lane), pb[j], acc[m]);
        }
      });
  };
  if (fixed_ref)
    run(std::integral_constant<bool, false>{});
  else
    run(std::integral_constant<bool, true>{});
  if (!valid) return;
  const float l = l_run + __shfl_xor(l_run, 32);
  store_acc<HD>(a.o + ((size_t)t * H + head) * HD, acc, l > 0.f ? (DROP ? a.drop.inv_keep : 1.f) / l : 0.f, h);
  if (h == 0) a.lse_out[(size_t)head * a.total_q + t] = l > 0.f ? (a.c * m_run + fast_log2(l)) * kLn2 : -INFINITY;
}

// ------------------------------------------------------------------ dQ pass
// Queries on lanes: S^T = K q^T, dP^T = V dO^T, P = exp2(c S - LSE2),
// dS = P (dP - D), dQ^T += K^T dS^T.  Also writes the dK/dV pass's row
// statistics {-LSE2 / c, -D} of its queries.
template <int HD, bool DROP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(HD == 64 && !DROP ? ESA_WIDE_WAVES_DQ64 : 1)))
void wide_dq_kernel(const WideArgs a) {
  constexpr int HP = (HD + 31) / 32 * 32, NC = (HD + 15) / 16, NM = HP / 32, NO = HP / 8;
  __shared__ __align__(16) bf16 sK[2][NO * kWTokPad * 8];
  __shared__ __align__(16) bf16 sV[2][NO * kWTokPad * 8];
  __shared__ __align__(16) uint32_t sKey[2][DROP ? kWStage : 4];   // column keys of the staged keys
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, h = lane >> 5;
  const int H = a.heads;
  int item, head;
  wide_item_head<HD>(H, item, head);
  if (item >= *a.count) return;
  const int4 g = a.groups[item];
  const int t = g.x + wave * kTile + col;
  const bool valid = t < g.y, active = g.x + wave * kTile < g.y;
  const size_t row = ((size_t)(valid ? t : g.x) * H + head) * HD;
  bf16x8 qop[NC], gop[NC];
  float dsum = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    qop[c] = row_op<HD>(a.q + row, 2 * c + h);
    gop[c] = row_op<HD>(a.dout + row, 2 * c + h);
    const bf16x8 o = row_op<HD>(a.out + row, 2 * c + h);
#pragma unroll
    for (int e = 0; e < 8; ++e) dsum = fmaf((float)gop[c][e], (float)o[e], dsum);
  }
  wide_zero_pad<HD>(sK[0], sK[1], sV[0], sV[1], tid);
  dsum += __shfl_xor(dsum, 32);
  const float lq = a.lse[(size_t)head * a.total_q + (valid ? t : g.x)];
  const float lse2 = lq == -INFINITY ? INFINITY : lq * kLog2e;   // rows without keys: P = 0
  if (valid && h == 0)
    a.aux[(size_t)head * a.tq_pad + t] = make_float2(lq == -INFINITY ? kDeadRow : -lse2 / a.c, -dsum);
  const uint32_t rk = DROP ? drop_row(a.drop, valid ? t : g.x, head) : 0u;
  f32x16 acc[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) acc[m] = f32x16{};
  const int n_tiles = (g.w - g.z + kTile - 1) >> 5;
  const int n_stages = (n_tiles + 1) >> 1;
  const f32x16 zero = {};
  wide_walk(
      n_stages,
      [&](int st) {
        WStageK<HD> s;
        s.rows = wide_gload<HD>(a.k, a.v, g.z + st * kWStage, a.total_k, H, head, tid);
        s.key = DROP && tid < kWStage ? drop_col(a.drop, g.z + st * kWStage + tid) : 0u;
        return s;
      },
      [&](int buf, const WStageK<HD>& s) {
        wide_lstore<HD>(sK[buf], sV[buf], s.rows, tid);
        if (DROP && tid < kWStage) sKey[buf][tid] = s.key;
      },
      [&](int buf, int st) {
        if (!active) return;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          if (2 * st + u >= n_tiles) break;
          const int k0 = g.z + st * kWStage + u * kTile;
          f32x16 s = zero, dp = zero;
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            s = mfma32(row_octet<NO>(sK[buf], u * kTile + kperm(col), 2 * c + h), qop[c], s);
            dp = mfma32(row_octet<NO>(sV[buf], u * kTile + kperm(col), 2 * c + h), gop[c], dp);
          }
          if (k0 + kTile > g.w) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = k0 + row_local(r, h) < g.w ? s[r] : -INFINITY;
          }
          float ds[16];
          if (DROP) {
            float dpk[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) dpk[r] = dp[r] * a.drop.inv_keep;
            drop_tile(a.drop, rk, &sKey[buf][u * kTile], h, g.z & 1, dpk);
#pragma unroll
            for (int r = 0; r < 16; ++r) ds[r] = fast_exp2(fmaf(s[r], a.c, -lse2)) * (dpk[r] - dsum);
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) ds[r] = fast_exp2(fmaf(s[r], a.c, -lse2)) * (dp[r] - dsum);
          }
#pragma unroll
          for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[m] = mfma32(tr_dims<NO>(sK[buf], m, 2 * u + j, lane), cvt8(ds + 8 * j), acc[m]);
        }
      });
  if (!valid) return;
  store_acc<HD>(a.dq + ((size_t)t * H + head) * HD, acc, a.scale, h);
}

// ------------------------------------------------------------------ dK/dV pass
// Keys on lanes, queries in rows: S = Q k^T - LSE2 / c and dP = dO v^T - D
// (the row statistics as accumulator seeds), P = exp2(c S), dS = P dP,
// dV^T += dO^T P, dK^T += Q^T dS.  A stage holds 64 queries' Q and dO rows
// and their statistics.
template <int HD, bool DROP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(ESA_WIDE_WAVES_DKDV > 0 ? ESA_WIDE_WAVES_DKDV : 1)))
void wide_dkdv_kernel(const WideArgs a) {
  constexpr int HP = (HD + 31) / 32 * 32, NC = (HD + 15) / 16, NM = HP / 32, NO = HP / 8;
  __shared__ __align__(16) bf16 sQ[2][NO * kWTokPad * 8];
  __shared__ __align__(16) bf16 sG[2][NO * kWTokPad * 8];
  __shared__ __align__(16) float sLse[2][kWStage], sDel[2][kWStage];
  __shared__ __align__(16) uint32_t sKey[2][DROP ? kWStage : 4];   // row keys of the staged queries
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, h = lane >> 5;
  const int H = a.heads;
  int item, head;
  wide_item_head<HD>(H, item, head);
  if (item >= *a.count) return;
  const int4 g = a.groups[item];   // outer = keys, inner = queries
  const int t = g.x + wave * kTile + col;
  const bool valid = t < g.y, active = g.x + wave * kTile < g.y;
  const size_t row = ((size_t)(valid ? t : g.x) * H + head) * HD;
  bf16x8 kop[NC], vop[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    kop[c] = row_op<HD>(a.k + row, 2 * c + h);
    vop[c] = row_op<HD>(a.v + row, 2 * c + h);
  }
  wide_zero_pad<HD>(sQ[0], sQ[1], sG[0], sG[1], tid);
  const uint32_t ck = DROP ? drop_col(a.drop, valid ? t : g.x) : 0u;
  f32x16 dva[NM], dka[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) dva[m] = dka[m] = f32x16{};
  const int n_tiles = (g.w - g.z + kTile - 1) >> 5;
  const int n_stages = (n_tiles + 1) >> 1;
  struct Stage { WStage<HD> rows; float2 st; uint32_t key; };
  wide_walk(
      n_stages,
      [&](int st) {
        Stage s;
        s.rows = wide_gload<HD>(a.q, a.dout, g.z + st * kWStage, a.total_q, H, head, tid);
        const int qi = g.z + st * kWStage + tid;
        s.st = tid < kWStage ? a.aux[(size_t)head * a.tq_pad + min(qi, a.tq_pad - 1)] : make_float2(0.f, 0.f);
        s.key = DROP && tid < kWStage ? drop_row(a.drop, qi, head) : 0u;
        return s;
      },
      [&](int buf, const Stage& s) {
        wide_lstore<HD>(sQ[buf], sG[buf], s.rows, tid);
        if (tid < kWStage) {
          sLse[buf][tid] = s.st.x;
          sDel[buf][tid] = s.st.y;
          if (DROP) sKey[buf][tid] = s.key;
        }
      },
      [&](int buf, int st) {
        if (!active) return;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          if (2 * st + u >= n_tiles) break;
          const int q0 = g.z + st * kWStage + u * kTile;
          // seeds: register r of lane (col, h) is query row_local(r, h) = 8 h + r (r < 8), 16 + 8 h + r - 8
          f32x16 s, dp;
#pragma unroll
          for (int b = 0; b < 2; ++b) {
            const f32x4 l0 = ldsf4(&sLse[buf][u * kTile + 16 * b + 8 * h]);
            const f32x4 l1 = ldsf4(&sLse[buf][u * kTile + 16 * b + 8 * h + 4]);
            const f32x4 d0 = ldsf4(&sDel[buf][u * kTile + 16 * b + 8 * h]);
            const f32x4 d1 = ldsf4(&sDel[buf][u * kTile + 16 * b + 8 * h + 4]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              s[8 * b + e] = l0[e]; s[8 * b + 4 + e] = l1[e];
              dp[8 * b + e] = d0[e]; dp[8 * b + 4 + e] = d1[e];
            }
          }
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            s = mfma32(row_octet<NO>(sQ[buf], u * kTile + kperm(col), 2 * c + h), kop[c], s);
            dp = mfma32(row_octet<NO>(sG[buf], u * kTile + kperm(col), 2 * c + h), vop[c], dp);
          }
          float p[16], ds[16];
#pragma unroll
          for (int r = 0; r < 16; ++r) p[r] = fast_exp2(s[r] * a.c);
          if (q0 + kTile > g.w) {   // the segment's last, partial query tile
#pragma unroll
            for (int r = 0; r < 16; ++r) p[r] = q0 + row_local(r, h) < g.w ? p[r] : 0.f;
          }
#pragma unroll
          for (int r = 0; r < 16; ++r) ds[r] = p[r] * dp[r];
          if (DROP) {
            // dp holds dO v - D: a kept partner's dS is P ((dO v) / (1 - p) - D), a dropped one's -P D
            float nd[16], pk[16];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
              const f32x4 d0 = ldsf4(&sDel[buf][u * kTile + 16 * b + 8 * h]);
              const f32x4 d1 = ldsf4(&sDel[buf][u * kTile + 16 * b + 8 * h + 4]);
#pragma unroll
              for (int e = 0; e < 4; ++e) { nd[8 * b + e] = d0[e]; nd[8 * b + 4 + e] = d1[e]; }
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) pk[r] = 1.f;
            drop_tile_key(a.drop, ck, &sKey[buf][u * kTile], h, t & 1, pk);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const bool keep = pk[r] != 0.f;
              ds[r] = p[r] * (keep ? fmaf(a.drop.inv_keep, dp[r] - nd[r], nd[r]) : nd[r]);
              p[r] = keep ? p[r] : 0.f;
            }
          }
#pragma unroll
          for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              dva[m] = mfma32(tr_dims<NO>(sG[buf], m, 2 * u + j, lane), cvt8(p + 8 * j), dva[m]);
              dka[m] = mfma32(tr_dims<NO>(sQ[buf], m, 2 * u + j, lane), cvt8(ds + 8 * j), dka[m]);
            }
        }
      });
  if (!valid) return;
  store_acc<HD>(a.dv + ((size_t)t * H + head) * HD, dva, DROP ? a.drop.inv_keep : 1.f, h);
  store_acc<HD>(a.dk + ((size_t)t * H + head) * HD, dka, a.scale, h);
}

// ------------------------------------------------------------------ prep
// Segment plans of both directions (128-token groups, longest partner range
// first) and, for the backward, the row statistics of the queries after the
// last segment up to the 32-row boundary (the dK/dV pass stages them; dead
// rows give P = 0).
struct WidePrep {
  const int* cu_q; const int* cu_k; int nseg;
  int total_q, total_k, heads, tq_pad, tk_tiles;
  int4* plan_q; int* count_q; int4* plan_k; int* count_k;
  float2* aux;
  const bf16* k; float* knorm;   // forward: max |k| per (head, 32-key tile)
  int nb_plan_k, nb_knorm, nb_rows;
};

// max |k_t| over key tile `tile` per head: knorm[h * n_tiles + tile].  Lanes
// read consecutive 16-byte chunks of the tile's rows (heads fastest), a row's
// C = HD / 8 chunks on C consecutive lanes summed by shuffles (head dim 24:
// a row per lane); with a power-of-two head count and H C <= 64 the rows of
// one head in a wave are then combined by shuffles too, so one LDS atomic per
// head and wave remains.  (A row per lane with eight 16-byte loads, each
// instruction touching 64 lines at hd 64, took 4x longer.)
template <int HD>
DEVI void wide_knorm_block(const WidePrep& p, int tile, int tid) {
  constexpr int C = (HD / 8 & (HD / 8 - 1)) == 0 ? HD / 8 : 1;   // chunks per lane group
  constexpr int CPL = HD / 8 / C;                                  // chunks per lane
  __shared__ int smax[256];
  const int H = p.heads, lane = tid & 63;
  for (int h0 = 0; h0 < H; h0 += 256) {
    const int hn = min(256, H - h0);
    const bool wave_heads = hn == H && (H & (H - 1)) == 0 && H * C <= 64;
    if (tid < hn) smax[tid] = 0;
    __syncthreads();
    const int items = kTile * hn * C;
    for (int i0 = 0; i0 < items; i0 += 256) {   // block-uniform trip count: every lane reaches the shuffles
      const int i = i0 + tid;
      const int rr = i / C, c = i - rr * C;
      const int t = tile * kTile + rr / hn, h = h0 + rr % hn;
      float x = 0.f;
      if (i < items && t < p.total_k) {
        const bf16x8* r = reinterpret_cast<const bf16x8*>(p.k + ((size_t)t * H + h) * HD) + c * CPL;
#pragma unroll
        for (int o = 0; o < CPL; ++o) {
          const bf16x8 u = r[o];
#pragma unroll
          for (int e = 0; e < 8; ++e) x = fmaf((float)u[e], (float)u[e], x);
        }
      }
#pragma unroll
      for (int o = 1; o < C; o <<= 1) x += __shfl_xor(x, o);   // the row's |k|^2 on all its lanes
      if (wave_heads) {
        for (int o = H * C; o < 64; o <<= 1) x = fmaxf(x, __shfl_xor(x, o));
        if (lane < H * C && c == 0 && i < items) atomicMax(&smax[h - h0], __float_as_int(x));
      } else if (c == 0 && i < items) {
        atomicMax(&smax[h - h0], __float_as_int(x));   // x >= 0: int order is float order
      }
    }
    __syncthreads();
    if (tid < hn) p.knorm[(size_t)(h0 + tid) * p.tk_tiles + tile] = sqrtf(__int_as_float(smax[tid]));
    __syncthreads();
  }
}

template <int HD>
__global__ __launch_bounds__(256) void wide_prep_kernel(const WidePrep p) {
  const int tid = threadIdx.x;
  int b = blockIdx.x;
  if (b == 0) { seg_plan_block(p.cu_q, p.cu_k, p.nseg, kWGroup, p.plan_q, p.count_q, tid); return; }
  b -= 1;
  if (b < p.nb_plan_k) { seg_plan_block(p.cu_k, p.cu_q, p.nseg, kWGroup, p.plan_k, p.count_k, tid); return; }
  b -= p.nb_plan_k;
  if (b < p.nb_knorm) { wide_knorm_block<HD>(p, b, tid); return; }
  b -= p.nb_knorm;
  const int t0 = min(max(p.cu_q[p.nseg], 0), p.total_q);
  const long n = (long)p.heads * (p.tq_pad - t0);
  for (long idx = (long)b * 256 + tid; idx < n; idx += (long)p.nb_rows * 256) {
    const int hh = (int)(idx % p.heads), t = t0 + (int)(idx / p.heads);
    p.aux[(size_t)hh * p.tq_pad + t] = make_float2(kDeadRow, -0.f);
  }
}

size_t wal256(size_t x) { return (x + 255) & ~size_t(255); }
int wr32(int x) { return (x + kTile - 1) / kTile * kTile; }
// Groups of one direction: at most ceil(T / 128) + (non-empty segments) <= ceil(T / 128) + T.
size_t wplan_bytes(int total) { return wal256(((size_t)(total + kWGroup - 1) / kWGroup + (size_t)total + 1) * 16); }

struct WideWs { size_t counts, plan_q, plan_k, aux, knorm, total; };
WideWs wide_ws(int total_q, int total_k, int heads, bool backward) {
  WideWs w{};
  size_t off = 0;
  w.counts = off; off += 256;
  w.plan_q = off; off += wplan_bytes(total_q);
  if (backward) {
    w.plan_k = off; off += wplan_bytes(total_k);
    w.aux = off; off += wal256((size_t)heads * wr32(total_q) * 8);
  } else {
    w.knorm = off; off += wal256((size_t)heads * (wr32(total_k) / kTile) * 4);
  }
  w.total = off;
  return w;
}

unsigned wide_grid(int total_outer, int nseg, int heads) {
  return (unsigned)(((total_outer + kWGroup - 1) / kWGroup + min(nseg, total_outer)) * heads);
}

#define ESA_WIDE_LAUNCH_HD(KERNEL, D, hd, grid, st, a)                                   \
  do {                                                                                    \
    if (hd == 16) hipLaunchKernelGGL((KERNEL<16, D>), grid, dim3(256), 0, st, a);         \
    else if (hd == 24) hipLaunchKernelGGL((KERNEL<24, D>), grid, dim3(256), 0, st, a);    \
    else if (hd == 32) hipLaunchKernelGGL((KERNEL<32, D>), grid, dim3(256), 0, st, a);    \
    else hipLaunchKernelGGL((KERNEL<64, D>), grid, dim3(256), 0, st, a);                  \
  } while (0)
#define ESA_WIDE_PREP(hd, grid, st, p)                                                         \
  do {                                                                                    \
    if (hd == 16) hipLaunchKernelGGL((wide_prep_kernel<16>), grid, dim3(256), 0, st, p);  \
    else if (hd == 24) hipLaunchKernelGGL((wide_prep_kernel<24>), grid, dim3(256), 0, st, p); \
    else if (hd == 32) hipLaunchKernelGGL((wide_prep_kernel<32>), grid, dim3(256), 0, st, p); \
    else hipLaunchKernelGGL((wide_prep_kernel<64>), grid, dim3(256), 0, st, p);           \
  } while (0)
// Head dim 16 only with dropout (without, esa_attn_dense.hip's kernels run).
#define ESA_WIDE_LAUNCH(KERNEL, hd, drop, grid, st, a)                                   \
  do {                                                                                    \
    if (drop) ESA_WIDE_LAUNCH_HD(KERNEL, true, hd, grid, st, a);                         \
    else ESA_WIDE_LAUNCH_HD(KERNEL, false, hd, grid, st, a);                             \
  } while (0)

}  // namespace

size_t wide_attn_workspace_size(int total_q, int total_k, int heads, int head_dim, bool backward) {
  (void)head_dim;
  return wide_ws(total_q, total_k, heads, backward).total;
}

int wide_attn_fwd(const DenseAttnCall& c, void* workspace, size_t workspace_bytes, hipStream_t st) {
  if (c.head_dim != 24 && c.head_dim != 32 && c.head_dim != 64 && !(c.head_dim == 16 && c.dropout))
    return ESA_ERR_HEAD_DIM;
  const WideWs w = wide_ws(c.total_q, c.total_k, c.heads, false);
  if (workspace_bytes < w.total) return ESA_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  WidePrep p{};
  p.cu_q = c.cu_q; p.cu_k = c.cu_k; p.nseg = c.nseg;
  p.total_q = c.total_q; p.total_k = c.total_k; p.heads = c.heads; p.tq_pad = wr32(c.total_q);
  p.tk_tiles = wr32(c.total_k) / kTile;
  p.count_q = reinterpret_cast<int*>(ws + w.counts);
  p.plan_q = reinterpret_cast<int4*>(ws + w.plan_q);
  p.k = static_cast<const bf16*>(c.k); p.knorm = reinterpret_cast<float*>(ws + w.knorm);
  p.nb_knorm = p.tk_tiles;
  ESA_TIMED(esa_profile::kAttnPrep, st, ESA_WIDE_PREP(c.head_dim, dim3(1 + p.nb_knorm), st, p));
  ESA_LAUNCH_CHECK();
  WideArgs a{};
  a.q = static_cast<const bf16*>(c.q); a.k = static_cast<const bf16*>(c.k); a.v = static_cast<const bf16*>(c.v);
  a.groups = p.plan_q; a.count = p.count_q;
  a.total_q = c.total_q; a.total_k = c.total_k; a.heads = c.heads; a.tq_pad = p.tq_pad;
  a.c = c.scale * kLog2e; a.scale = c.scale;
  a.drop = c.drop;
  a.knorm = p.knorm; a.tk_tiles = p.tk_tiles;
  a.o = static_cast<bf16*>(c.out); a.lse_out = c.lse;
  ESA_TIMED(esa_profile::kAttnFwd, st,
            ESA_WIDE_LAUNCH(wide_fwd_kernel, c.head_dim, c.dropout, dim3(wide_grid(c.total_q, c.nseg, c.heads)), st,
                            a));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}

int wide_attn_bwd(const DenseAttnCall& c, void* workspace, size_t workspace_bytes, hipStream_t st) {
  if (c.head_dim != 24 && c.head_dim != 32 && c.head_dim != 64 && !(c.head_dim == 16 && c.dropout))
    return ESA_ERR_HEAD_DIM;
  const WideWs w = wide_ws(c.total_q, c.total_k, c.heads, true);
  if (workspace_bytes < w.total) return ESA_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  WidePrep p{};
  p.cu_q = c.cu_q; p.cu_k = c.cu_k; p.nseg = c.nseg;
  p.total_q = c.total_q; p.heads = c.heads; p.tq_pad = wr32(c.total_q);
  p.count_q = reinterpret_cast<int*>(ws + w.counts);
  p.count_k = p.count_q + 1;
  p.plan_q = reinterpret_cast<int4*>(ws + w.plan_q);
  p.plan_k = reinterpret_cast<int4*>(ws + w.plan_k);
  p.aux = reinterpret_cast<float2*>(ws + w.aux);
  p.nb_plan_k = 1;
  p.nb_rows = (int)std::max(1L, ((long)c.heads * (p.tq_pad - c.total_q) + 255) / 256);
  ESA_TIMED(esa_profile::kAttnPrep, st, ESA_WIDE_PREP(c.head_dim, dim3(2 + p.nb_rows), st, p));
  ESA_LAUNCH_CHECK();
  WideArgs a{};
  a.q = static_cast<const bf16*>(c.q); a.k = static_cast<const bf16*>(c.k); a.v = static_cast<const bf16*>(c.v);
  a.out = static_cast<const bf16*>(c.out_in); a.dout = static_cast<const bf16*>(c.dout);
  a.lse = c.lse_in; a.aux = p.aux;
  a.total_q = c.total_q; a.total_k = c.total_k; a.heads = c.heads; a.tq_pad = p.tq_pad;
  a.c = c.scale * kLog2e; a.scale = c.scale;
  a.drop = c.drop;
  a.dq = static_cast<bf16*>(c.dq); a.dk = static_cast<bf16*>(c.dk); a.dv = static_cast<bf16*>(c.dv);
  // dQ first: it writes the row statistics the dK/dV pass stages
  a.groups = p.plan_q; a.count = p.count_q;
  ESA_TIMED(esa_profile::kAttnBwdDq, st,
            ESA_WIDE_LAUNCH(wide_dq_kernel, c.head_dim, c.dropout, dim3(wide_grid(c.total_q, c.nseg, c.heads)), st,
                            a));
  ESA_LAUNCH_CHECK();
  a.groups = p.plan_k; a.count = p.count_k;
  ESA_TIMED(esa_profile::kAttnBwdDkdv, st,
            ESA_WIDE_LAUNCH(wide_dkdv_kernel, c.head_dim, c.dropout, dim3(wide_grid(c.total_k, c.nseg, c.heads)), st,
                            a));
  ESA_LAUNCH_CHECK();
  return ESA_OK;
}
