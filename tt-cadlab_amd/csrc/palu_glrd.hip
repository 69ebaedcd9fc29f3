// Fused decode over grouped latents with V rebuilt in-kernel (G-LRD): heads_per_group KV heads share
// one K latent and one V latent of rank up to 512, and every KV head has its own 128-column slices of
// U_k and U_v (palu_sdpa_decode with u_v; docs/superpowers/specs/2026-09-12-palu-tt-stage2b-design.md:
// 120-142, fp32 model palu_tt/fused.py:82-107 with u_v).
//
// Three launches on the caller's stream:
//   1. Scores. One workgroup per (row, KV head, sequence split), 4 waves (one per SIMD) that each take
//      their own pairs of 32-position blocks (no barrier in the loop). The KV head's whole u_k^T sits in
//      LDS as ready MFMA A tiles; the K latent streams from HBM straight into registers (tiled layout:
//      every load is one operand tile), a ring of rank blocks in flight. A wave rebuilds K^T (128 dims x
//      64 positions) on v_mfma_f32_16x16x32_bf16, rotates it in-lane (pair-relative RoPE table in
//      registers, query rotated back by the pair base) and contracts it with its query heads. The
//      scores go to the workspace as fp32 [block][head][32], already scaled by scale * log2 e.
//   2. Latent PV. One workgroup per (row, latent group, 16-head tile, sequence split); all query heads
//      of a group share the V latent, so the PV MFMA has the group's heads as its N dimension. The waves
//      split the V tiles and the blocks of the split, run the online softmax (exp2 domain, lazy
//      rescale) and accumulate O_lat^T = V_lat^T P^T for their V tiles, streamed from HBM two blocks
//      ahead. Partials (O_lat, m, l) per head and split go to the workspace.
//   3. Merge and V rebuild. One workgroup per (row, KV head, query head): log-sum-exp merge of the splits, then
//      out = O_lat u_v[h] / l in fp32 -- the same sum as softmax(q K^T) (V_lat u_v[h]), V never built.
// The K latent of a group is read by heads_per_group scores workgroups; they are numbered so they land
// on one XCD (the dispatcher deals consecutive workgroup ids round-robin over the 8 XCDs) and meet in
// its L2.
#include "palu_glrd_scores.h"

namespace {

constexpr int G_NW = 8;                 // waves per workgroup (PV kernel)
constexpr int G_PSTRIDE_PAD = 4;        // partial row: r_v values, m, l, 2 pad (16-byte rows)
constexpr int G_MAX_SPLITS2 = 128;      // PV splits per group (the merge workgroup stages their weights)

inline int glrd_pv_splits(int items2, int nb) {
  // About 256 PV workgroups, at least 4 blocks each, at most 128 splits.
  int s = (256 + items2 - 1) / items2;
  const int cap = (nb + 3) / 4 < 128 ? (nb + 3) / 4 : 128;
  s = s < cap ? s : cap;
  return s < 1 ? 1 : s;
}

struct GlrdPlan {
  int n_ht, n_splits2, split_len2, n_wg2;
  size_t scores_floats, part_floats;
};

// Workspace sizing: the PV pass's split partials are counted as if every group had n_splits2 splits
// (the per-group plan below hands out the same total).
inline GlrdPlan glrd_plan(int B, int n_q, int n_kv, int n_groups, int S, int rv) {
  GlrdPlan p;
  (void)n_kv;
  const int QH = n_q / n_groups;
  p.n_ht = (QH + 15) / 16;
  const int nb = (S + BLK - 1) / BLK;
  const int s2 = glrd_pv_splits(B * n_groups * p.n_ht, nb);
  p.split_len2 = ((nb + s2 - 1) / s2) * BLK;
  p.n_splits2 = (nb * BLK + p.split_len2 - 1) / p.split_len2;
  p.n_wg2 = B * n_groups * p.n_ht * p.n_splits2;
  p.scores_floats = (size_t)B * n_q * nb * BLK;
  p.part_floats = (size_t)B * n_q * p.n_splits2 * (rv + G_PSTRIDE_PAD);
  return p;
}

__host__ __device__ inline int glrd_pv_tg_group(int vt_g, int tpw);

// The PV pass's splits per group. A group of lower V rank covers its tiles with fewer tile groups and
// walks its blocks with more position groups, so it finishes a split sooner: the n_groups * n_splits2
// splits of the uniform plan are dealt out in proportion to each group's time per position (tile groups
// x (V tiles of its busiest wave + 2 for the scores and the softmax)), largest remaining share first, so
// one chip-fill of workgroups ends together. Equal ranks keep the uniform plan. Fills a.gns2 / gsl2 /
// gwg2 / gprow; returns the partial rows written. tpw: V tiles per wave of the launch.
inline int glrd_group_plan(DecodeArgs& a, const GlrdPlan& p, int tpw) {
  const int n_groups = a.n_kv / a.hpg;
  const int QH = a.hpg * a.rep;
  const int nb = (a.S + BLK - 1) / BLK;
  const int cap = (nb + 3) / 4 < G_MAX_SPLITS2 ? ((nb + 3) / 4 < 1 ? 1 : (nb + 3) / 4) : G_MAX_SPLITS2;
  int s[MAX_GROUPS], wt[MAX_GROUPS];
  bool uniform = true;
  for (int g = 0; g < n_groups; ++g) {
    s[g] = 1;
    uniform = uniform && a.grv[g] == a.grv[0];
    const int vt = a.grv[g] >> 4;
    wt[g] = glrd_pv_tg_group(vt, tpw) * ((vt < tpw ? vt : tpw) + 2);
  }
  if (uniform)
    for (int g = 0; g < n_groups; ++g) s[g] = p.n_splits2;
  for (int k = uniform ? n_groups * p.n_splits2 : n_groups; k < n_groups * p.n_splits2; ++k) {
    int best = -1;
    for (int g = 0; g < n_groups; ++g)      // largest weight / splits, compared without division
      if (s[g] < cap && (best < 0 || (long long)wt[g] * s[best] > (long long)wt[best] * s[g])) best = g;
    if (best < 0) break;
    ++s[best];
  }
  int wg = 0, row = 0;
  for (int g = 0; g < n_groups; ++g) {
    const int len = ((nb + s[g] - 1) / s[g]) * BLK;
    const int ns = (nb * BLK + len - 1) / len;      // <= s[g]
    a.gsl2[g] = len;
    a.gns2[g] = (short)ns;
    a.gwg2[g] = wg;
    a.gprow[g] = row;
    wg += a.B * p.n_ht * ns;
    row += a.B * QH * ns;
  }
  a.gwg2[n_groups] = wg;
  return row;                                       // partial rows the plan writes
}

// ---------------------------------------------------------------------------------------------------
// Pass 2: latent PV. The 8 waves form TG tile groups x PG position groups (TG * PG = 8): wave (tg, pg)
// owns V tiles tg * TPW .. tg * TPW + TPW - 1 and the blocks j = pg, pg + PG, ... of the split, with its
// own online softmax; the PG partials of a tile group are merged through LDS at the end. A block's
// scores are thus loaded and exponentiated by TG waves, not by all 8. TPW comes from the cache width (TG
// the smallest power of two with TG * 8 >= r_v / 16); a group of lower V rank takes the fewest tile
// groups that cover its own tiles, so its spare waves take more position groups instead of idling.
__host__ __device__ inline int glrd_pv_tg(int vt) {
  int tg = 1;
  while (tg * 8 < vt) tg *= 2;
  return tg;
}
// Tile groups of a group with vt_g V tiles when a wave holds tpw tiles.
__host__ __device__ inline int glrd_pv_tg_group(int vt_g, int tpw) {
  int tg = 1;
  while (tg * tpw < vt_g && tg < G_NW) tg *= 2;
  return tg;
}
__host__ __device__ inline int glrd_pv_lds(int tpw) { return G_NW * (16 * tpw * 16 + 2 * 16) * 4; }

template <int TPW, bool ROWS>
__global__ __launch_bounds__(G_NW * 64) void palu_glrd_pv_kernel(const DecodeArgs a, const float* scores, float* part,
                                                                 int n_ht) {
  static_assert(!ROWS || TPW % 2 == 0, "a ROWS wave loads its V tiles in 32-column pieces");
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int n_groups = a.n_kv / a.hpg;
  const int QH = a.hpg * a.rep;
  const int NB = (a.S + BLK - 1) / BLK;
  // workgroup -> (group, row, head tile, split): each group's workgroups form one range (per-group plan)
  int L = blockIdx.x;
  int grp = 0;
  while (grp + 1 < n_groups && L >= a.gwg2[grp + 1]) ++grp;
  L -= a.gwg2[grp];
  const int n_splits2 = a.gns2[grp], split_len2 = a.gsl2[grp];
  const int split = L % n_splits2;
  L /= n_splits2;
  const int ht = L % n_ht;
  const int b = L / n_ht;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int rv_g = a.grv[grp];                            // this group's rank: V tiles past it are never read
  const int VT = rv_g >> 4;
  const int TG = glrd_pv_tg_group(VT, TPW), PG = G_NW / TG;
  const int tg = w % TG, pg = w / TG;
  const int head = ht * 16 + n;                       // head of this lane column inside the group
  const bool head_live = head < QH;
  const int head_c = head_live ? head : QH - 1;

  int len = a.cur_pos[b] + 1;
  len = len < 0 ? 0 : (len > a.S ? a.S : len);
  const int s_lo = split * split_len2;
  const int s_hi = min(len, s_lo + split_len2);
  const int nblk = s_hi > s_lo ? (s_hi - s_lo + BLK - 1) / BLK : 0;
  const int nfull = s_hi > s_lo ? (s_hi - s_lo) / BLK : 0;

  const float* sc0 = scores + ((long long)(b * n_groups + grp) * NB + (s_lo >> 5)) * QH * BLK +
                     (long long)head_c * BLK + 8 * g;
  const long long blk_stride = (long long)QH * BLK;
  const int vw = a.gvw[grp];                              // the group's stream width
  const __bf16* vstream = a.v + b * a.v_sb + a.gvo[grp];
  const __bf16* vbase = vstream + (long long)(s_lo >> 5) * (32 * vw) + lane * 8;

  struct Blk {
    float4 s[2];             // positions 8g .. 8g+7 of this lane's head
    bf16x8 v[TPW];
  };
  // Loads of block j (past the split's data: its first block, unused; tiles past r_v: not loaded).
  // TILED: x.v[i] is V tile tg * TPW + i of the block, the A operand of the PV product as it stands.
  // ROWS: x.v[2 i2 + c] holds columns 32 (tg * TPW / 2 + i2) + 8 g .. +7 of position 8 (n / 4) + 4 c + n % 4
  // (rows past the cache end clamped to its last row, masked below); the step regroups each pair into
  // the two 16-column tiles of that 32-column piece.
  auto load = [&](int j, Blk& x) {
    const int jj = j < nblk ? j : 0;
    const float* p0 = sc0 + jj * blk_stride;
    x.s[0] = *reinterpret_cast<const float4*>(p0);
    x.s[1] = *reinterpret_cast<const float4*>(p0 + 4);
    // The V latent is read once per decode step (one workgroup per row, group and split): nontemporal.
    // Tiles past the group's rank are not loaded (their products are skipped below).
    if constexpr (ROWS) {
      const int pb = s_lo + jj * BLK;
#pragma unroll
      for (int i2 = 0; i2 < TPW / 2; ++i2) {
        const int piece = tg * (TPW / 2) + i2;
        if (2 * piece < VT) {
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const int p = min(pb + 8 * (n >> 2) + 4 * c + (n & 3), a.S - 1);
            // cached: the 64-byte piece is half a 128-byte line whose other half another tile group
            // reads (a nontemporal read would fetch the line twice)
            const uint32_t off = (uint32_t)(p * vw + 32 * piece + 8 * g) * 2u;   // 32-bit byte offset
            x.v[2 * i2 + c] = *reinterpret_cast<const bf16x8*>(reinterpret_cast<const char*>(vstream) + off);
          }
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        const int mt = tg * TPW + i;
        if (mt < VT)
          x.v[i] = __builtin_nontemporal_load(
              reinterpret_cast<const bf16x8*>(vbase + (long long)jj * (32 * vw) + mt * 512));
      }
    }
  };
  // ROWS: identity B operands; mfma16(row piece, idB[par]) moves 16 columns of a 32-column piece of
  // 16 positions into the accumulator layout, exactly (products with 1 and 0 in fp32).
  bf16x8 idB[ROWS ? 2 : 1];
  if constexpr (ROWS) {
#pragma unroll
    for (int par = 0; par < 2; ++par)
#pragma unroll
      for (int e = 0; e < 8; ++e) idB[par][e] = (8 * g + e == 16 * par + n) ? (__bf16)1.0f : (__bf16)0.0f;
  }

  f32x4 O[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) O[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = NEG_INF, l_run = 0.f;

  auto step = [&](auto partial_tag, int j, const Blk& x) __attribute__((always_inline)) {
    constexpr bool partial = decltype(partial_tag)::value;
    const int base = s_lo + j * BLK;
    float s[8] = {x.s[0].x, x.s[0].y, x.s[0].z, x.s[0].w, x.s[1].x, x.s[1].y, x.s[1].z, x.s[1].w};
    if constexpr (partial) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (base + 8 * g + e >= s_hi) s[e] = NEG_INF;
    }
    float bm = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
    bm = wave_max_xor48(bm);
    const bool need = __any(bm > m_run + LAZY_RESCALE_LOG2);
    const float mn = need ? fmaxf(m_run, bm) : m_run;
    const float alpha = need ? ((m_run == NEG_INF) ? 0.f : __builtin_amdgcn_exp2f(m_run - mn)) : 1.f;
#pragma unroll
    for (int i = 0; i < TPW; ++i) O[i] *= alpha;
    l_run *= alpha;
    m_run = mn;
    const float mref = (m_run == NEG_INF) ? 0.f : m_run;
    bf16x8 pB;
    float lsum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = head_live ? __builtin_amdgcn_exp2f(s[e] - mref) : 0.f;
      lsum += p;
      pB[e] = (__bf16)p;
    }
    l_run += lsum;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      if (tg * TPW + i >= VT) continue;              // past the group's rank (uniform)
      bf16x8 vA;
      if constexpr (ROWS) {
        // positions 8 g .. 8 g + 3 (half-block 0) and 8 g + 4 .. + 7 (half-block 1) of column 16 (tg TPW + i) + n
        f32x4 x0 = mfma16(x.v[2 * (i >> 1)], idB[i & 1], f32x4{0.f, 0.f, 0.f, 0.f});
        f32x4 x1 = mfma16(x.v[2 * (i >> 1) + 1], idB[i & 1], f32x4{0.f, 0.f, 0.f, 0.f});
        if constexpr (partial) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (base + 8 * g + e >= s_hi) x0[e] = 0.f;
            if (base + 8 * g + 4 + e >= s_hi) x1[e] = 0.f;
          }
        }
        vA = pack8(x0, x1);
      } else {
        vA = x.v[i];
        if constexpr (partial) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (base + 8 * g + e >= s_hi) vA[e] = (__bf16)0.0f;
        }
      }
      O[i] = mfma16(vA, pB, O[i]);
    }
  };

  const std::integral_constant<bool, false> full_blk;
  const std::integral_constant<bool, true> partial_blk;
  Blk x0, x1;
  load(pg, x0);
  load(pg + PG, x1);
  int j = pg;
  for (; j + PG < nfull; j += 2 * PG) {
    step(full_blk, j, x0);
    load(j + 2 * PG, x0);
    step(full_blk, j + PG, x1);
    load(j + 3 * PG, x1);
  }
  if (j < nfull) {
    step(full_blk, j, x0);
    j += PG;
    if (j < nblk) step(partial_blk, j, x1);         // then j == nfull: the partial last block
  } else if (j < nblk) {
    step(partial_blk, j, x0);
  }
  l_run = wave_sum_xor48(l_run);                      // over the wave's 4 position groups

  // merge the PG position groups of every tile group: wave w's partial in LDS, [16 heads][TPW * 16]
  // columns plus (m, l) per head
  float* ow = reinterpret_cast<float*>(smem) + w * (16 * TPW * 16 + 32);
#pragma unroll
  for (int i = 0; i < TPW; ++i)
    *reinterpret_cast<float4*>(ow + n * (TPW * 16) + 16 * i + 4 * g) = make_float4(O[i][0], O[i][1], O[i][2], O[i][3]);
  if (g == 0) { ow[16 * TPW * 16 + n] = m_run; ow[16 * TPW * 16 + 16 + n] = l_run; }
  __syncthreads();
  const int ncols = TG * TPW * 16;                    // >= r_v
  for (int e = tid; e < 16 * ncols; e += G_NW * 64) {
    const int hh = e / ncols, col = e - hh * ncols;
    const int t = col / (TPW * 16), c = col - t * (TPW * 16);
    if (ht * 16 + hh >= QH || col >= rv_g) continue;
    float M = NEG_INF;
    for (int q = 0; q < PG; ++q) M = fmaxf(M, reinterpret_cast<const float*>(smem)[(q * TG + t) * (16 * TPW * 16 + 32) + 16 * TPW * 16 + hh]);
    float acc = 0.f, Ls = 0.f;
    if (M != NEG_INF) {
      for (int q = 0; q < PG; ++q) {
        const float* oq = reinterpret_cast<const float*>(smem) + (q * TG + t) * (16 * TPW * 16 + 32);
        const float f = __builtin_amdgcn_exp2f(oq[16 * TPW * 16 + hh] - M);
        acc += oq[hh * (TPW * 16) + c] * f;
        Ls += oq[16 * TPW * 16 + 16 + hh] * f;
      }
    }
    const int row = a.gprow[grp] + (b * QH + ht * 16 + hh) * n_splits2 + split;
    float* prow = part + (long long)row * (a.rv + G_PSTRIDE_PAD);
    prow[col] = acc;
    if (col == 0) { prow[a.rv] = M; prow[a.rv + 1] = Ls; }
  }
}

// ---------------------------------------------------------------------------------------------------
// Pass 3: merge the splits of one query head of one (row, KV head) and apply u_v; one workgroup per
// (row, KV head, query head), so the launch has B * n_kv * rep workgroups (512 at the benchmark's
// shapes) instead of one per (row, KV head). The split weights 2^(m_s - M) are computed once, each latent
// column of O_lat is merged once (a dot product over independent loads), and the projection reads u_v
// in 16-byte pieces: thread (rank slice, 8 output dims) accumulates 8 outputs over its slice; the 16
// slices are summed through LDS.

// Dynamic LDS: red [16 rank slices][HD], olat [rv], wsplit [G_MAX_SPLITS2], lsum.
__host__ __device__ inline int glrd_out_lds(int rv) { return (16 * HD + rv + G_MAX_SPLITS2 + 4) * 4; }

template <typename OutT>
__global__ __launch_bounds__(256) void palu_glrd_out_kernel(const DecodeArgs a, const float* part) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int item = blockIdx.x, h = blockIdx.y;        // query head h of the item's KV head
  const int b = item / a.n_kv, kvh = item - b * a.n_kv;
  const int grp = kvh / a.hpg;
  const int rv = a.grv[grp];                          // the group's rank: partial columns past it are unset
  const int n_splits2 = a.gns2[grp];
  float* red = reinterpret_cast<float*>(smem);
  float* olat = red + 16 * HD;
  float* wsplit = olat + a.rv;
  float* lsum = wsplit + G_MAX_SPLITS2;
  const int stride = a.rv + G_PSTRIDE_PAD;
  const int tid = threadIdx.x;
  const int hh = (kvh - grp * a.hpg) * a.rep + h;     // query head within the group
  const float* ph = part + (long long)(a.gprow[grp] + (b * a.hpg * a.rep + hh) * n_splits2) * stride;
  // split weights: wsplit[s] = 2^(m_s - M); lsum = sum_s l_s 2^(m_s - M). The first wave's lanes take
  // the splits in turn.
  if (tid < 64) {
    const int lane = tid;
    float M = NEG_INF;
    for (int s = lane; s < n_splits2; s += 64) M = fmaxf(M, ph[(long long)s * stride + a.rv]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    float Ls = 0.f;
    for (int s = lane; s < n_splits2; s += 64) {
      const float f = (M == NEG_INF) ? 0.f : __builtin_amdgcn_exp2f(ph[(long long)s * stride + a.rv] - M);
      wsplit[s] = f;
      Ls += ph[(long long)s * stride + a.rv + 1] * f;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) Ls += __shfl_xor(Ls, o, 64);
    if (lane == 0) lsum[0] = Ls;
  }
  __syncthreads();
  for (int r = tid; r < rv; r += 256) {
    const float* pr = ph + r;
    float acc = 0.f;
#pragma unroll 8
    for (int s = 0; s < n_splits2; ++s) acc += pr[(long long)s * stride] * wsplit[s];
    olat[r] = acc;
  }
  __syncthreads();
  const int dg = tid & 15, rs = tid >> 4;             // 8 output dims, one of 16 rank slices
  const int per = rv / 16;                              // rv is a multiple of 32
  const __bf16* uv = a.u_v + (long long)kvh * a.rv * HD + 8 * dg;
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
#pragma unroll 8                                        // 8 u_v rows in flight
  for (int r = rs * per; r < rs * per + per; ++r) {
    const bf16x8 u = *reinterpret_cast<const bf16x8*>(uv + (long long)r * HD);
    const float o = olat[r];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] += o * (float)u[j];
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) red[rs * HD + 8 * dg + j] = acc[j];
  __syncthreads();
  if (tid < HD) {
    float sum = 0.f;
#pragma unroll
    for (int q = 0; q < 16; ++q) sum += red[q * HD + tid];
    const float Ls = lsum[0];
    OutT* o = static_cast<OutT*>(a.out) + out_index(a, b, ((long long)kvh * a.rep + h) * HD + tid, (long long)a.n_q * HD);
    store_out(o, Ls > 0.f ? sum / Ls : 0.f);
  }
}


template <typename TabT, bool ROWS>
int scores_full_kb(const DecodeArgs& a, float* scores, int n_wg, hipStream_t s) {
  switch ((a.rk_eff / 32 + 1) / 2) {              // the launch's rank blocks rounded up to even
    case 1:
    case 2:
    case 3:
    case 4: return palu::glrd_scores_narrow(a, scores, n_wg, s, ROWS, std::is_same<TabT, float>::value);
    case 5: return launch_scores_full<10, TabT, ROWS>(a, scores, n_wg, s);
    case 6: return launch_scores_full<12, TabT, ROWS>(a, scores, n_wg, s);
    case 7: return launch_scores_full<14, TabT, ROWS>(a, scores, n_wg, s);
    case 8: return launch_scores_full<16, TabT, ROWS>(a, scores, n_wg, s);
  }
  return fail(PALU_EUNSUPPORTED, "grouped-latent r_k %d (32 .. 512 in steps of 32)", a.rk_eff);
}

template <typename K>
int set_out_lds(K kern, int lds) {
  static int attr_set = 0;                 // one static per kernel instantiation
  if (attr_set < lds) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return fail(PALU_EHIP, "hipFuncSetAttribute: %s", hipGetErrorString(e));
    attr_set = lds;
  }
  return PALU_OK;
}

template <int TPW, bool ROWS>
int launch_pv_t(const DecodeArgs& a, const float* scores, float* part, const GlrdPlan& p, hipStream_t s) {
  const int lds = glrd_pv_lds(TPW);
  auto kern = palu_glrd_pv_kernel<TPW, ROWS>;
  static int attr_set = 0;
  if (attr_set < lds) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return fail(PALU_EHIP, "hipFuncSetAttribute: %s", hipGetErrorString(e));
    attr_set = lds;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)a.gwg2[a.n_kv / a.hpg]), dim3(G_NW * 64), lds, s, a, scores, part, p.n_ht);
  return PALU_OK;
}

// V tiles per wave: the tile groups' share of the cache width's tiles; ROWS rounds it up to even (a
// wave's tiles are whole 32-column pieces of the rows). The kernel derives the same tile groups.
inline int glrd_pv_tpw(int rv, bool rows) {
  const int vt = rv >> 4;
  const int tpw = (vt + glrd_pv_tg(vt) - 1) / glrd_pv_tg(vt);
  return rows ? (tpw + 1) & ~1 : tpw;
}

int launch_pv(const DecodeArgs& a, const float* scores, float* part, const GlrdPlan& p, bool rows, hipStream_t s) {
  if (rows) {
    switch (glrd_pv_tpw(a.rv, true)) {
      case 2: return launch_pv_t<2, true>(a, scores, part, p, s);
      case 4: return launch_pv_t<4, true>(a, scores, part, p, s);
      case 6: return launch_pv_t<6, true>(a, scores, part, p, s);
      case 8: return launch_pv_t<8, true>(a, scores, part, p, s);
    }
  } else {
    switch (glrd_pv_tpw(a.rv, false)) {
      case 1: return launch_pv_t<1, false>(a, scores, part, p, s);
      case 2: return launch_pv_t<2, false>(a, scores, part, p, s);
      case 3: return launch_pv_t<3, false>(a, scores, part, p, s);
      case 4: return launch_pv_t<4, false>(a, scores, part, p, s);
      case 5: return launch_pv_t<5, false>(a, scores, part, p, s);
      case 6: return launch_pv_t<6, false>(a, scores, part, p, s);
      case 7: return launch_pv_t<7, false>(a, scores, part, p, s);
      case 8: return launch_pv_t<8, false>(a, scores, part, p, s);
    }
  }
  return fail(PALU_EUNSUPPORTED, "grouped-latent r_v %d (32 .. 512 in steps of 32)", a.rv);
}

}  // namespace

namespace palu {

size_t glrd_workspace_bytes(int batch, int n_q, int n_kv, int n_groups, int seq_len, int r_v) {
  if (batch <= 0 || n_q <= 0 || n_kv <= 0 || n_groups <= 0 || seq_len <= 0 || r_v <= 0 || n_kv % n_groups) return 0;
  const GlrdPlan p = glrd_plan(batch, n_q, n_kv, n_groups, seq_len, r_v);
  return (p.scores_floats + p.part_floats) * sizeof(float) + 256;
}

int dispatch_glrd(const DecodeArgs& a0, bool rows, int cs_dtype, int out_dtype, hipStream_t s) {
  DecodeArgs a = a0;
  const int n_groups = a.n_kv / a.hpg;
  if (a.hpg * a.rep > 128)
    return fail(PALU_EUNSUPPORTED, "grouped latents with %d query heads per group (max 128)", a.hpg * a.rep);
  const GlrdPlan p = glrd_plan(a.B, a.n_q, a.n_kv, n_groups, a.S, a.rv);
  if (p.n_splits2 > G_MAX_SPLITS2) return fail(PALU_EUNSUPPORTED, "grouped-latent PV plan of %d splits", p.n_splits2);
  const size_t need = glrd_workspace_bytes(a.B, a.n_q, a.n_kv, n_groups, a.S, a.rv);
  if (a.ws == nullptr || a.ws_bytes < need)
    return fail(PALU_EINVAL, "workspace of %zu bytes needed (palu_glrd_workspace_bytes), got %zu", need, a.ws_bytes);
  float* scores = reinterpret_cast<float*>((reinterpret_cast<uintptr_t>(a.ws) + 255) & ~uintptr_t(255));
  float* part = scores + p.scores_floats;
  // Scores: one launch over every group when they share a K rank, else one launch per group at its own
  // rank (the kernel's rank loop is unrolled per width).
  bool uniform_k = true;
  for (int g = 0; g < n_groups; ++g) uniform_k = uniform_k && a.grk[g] == a.rk;
  hipError_t e = hipSuccess;
  for (int g0 = 0; g0 < n_groups; g0 += uniform_k ? n_groups : 1) {
    DecodeArgs ag = a;
    ag.grp_lo = g0;
    ag.grp_cnt = uniform_k ? n_groups : 1;
    ag.rk_eff = a.grk[g0];
    const Plan pf = plan_splits(a.B * ag.grp_cnt * a.hpg, a.S, 2 * G2_NW);
    ag.split_len = pf.split_len;
    ag.n_splits = pf.n_splits;
    const int n_wg = ((a.B * ag.grp_cnt * pf.n_splits + 7) / 8) * 8 * a.hpg;
    const int rc = rows ? (cs_dtype == PALU_DTYPE_F32 ? scores_full_kb<float, true>(ag, scores, n_wg, s)
                                                     : scores_full_kb<__bf16, true>(ag, scores, n_wg, s))
                        : (cs_dtype == PALU_DTYPE_F32 ? scores_full_kb<float, false>(ag, scores, n_wg, s)
                                                     : scores_full_kb<__bf16, false>(ag, scores, n_wg, s));
    if (rc) return rc;
    e = hipGetLastError();
    if (e != hipSuccess) return fail(PALU_EHIP, "grouped-latent scores kernel launch: %s", hipGetErrorString(e));
  }
  // the plan deals out the uniform plan's splits, so its partial rows fit the workspace's
  if ((size_t)glrd_group_plan(a, p, glrd_pv_tpw(a.rv, rows)) * (a.rv + G_PSTRIDE_PAD) > p.part_floats)
    return fail(PALU_EUNSUPPORTED, "grouped-latent PV plan exceeds its workspace");
  if (int rc2 = launch_pv(a, scores, part, p, rows, s)) return rc2;
  e = hipGetLastError();
  if (e != hipSuccess) return fail(PALU_EHIP, "grouped-latent PV kernel launch: %s", hipGetErrorString(e));
  const int out_lds = glrd_out_lds(a.rv);
  const dim3 out_grid((unsigned)(a.B * a.n_kv), (unsigned)a.rep);
  if (out_dtype == PALU_DTYPE_F32) {
    if (int rc3 = set_out_lds(palu_glrd_out_kernel<float>, out_lds)) return rc3;
    hipLaunchKernelGGL(palu_glrd_out_kernel<float>, out_grid, dim3(256), out_lds, s, a, part);
  } else {
    if (int rc3 = set_out_lds(palu_glrd_out_kernel<__bf16>, out_lds)) return rc3;
    hipLaunchKernelGGL(palu_glrd_out_kernel<__bf16>, out_grid, dim3(256), out_lds, s, a, part);
  }
  e = hipGetLastError();
  if (e != hipSuccess) return fail(PALU_EHIP, "grouped-latent output kernel launch: %s", hipGetErrorString(e));
  return PALU_OK;
}

}  // namespace palu
