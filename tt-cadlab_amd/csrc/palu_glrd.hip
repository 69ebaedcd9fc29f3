// Fused decode over grouped latents with V rebuilt in-kernel (G-LRD): heads_per_group KV heads share
// one K latent and one V latent of rank up to 512, and every KV head has its own 128-column slices of
// U_k and U_v (palu_sdpa_decode with u_v; docs/superpowers/specs/2026-09-12-palu-tt-stage2b-design.md:
// 120-142, fp32 model palu_tt/fused.py:82-107 with u_v).
//
// Shape of the kernel (one workgroup = one (row, KV head) item and one sequence split, 8 waves, two
// per SIMD):
//   * The 8 waves split the head dim: wave w owns dims 16w .. 16w+15 and keeps that 16 x r_k slice of
//     u_k^T in registers for the whole kernel (64 VGPRs at r_k = 512), so U_k is read once per
//     workgroup, whatever r_k. The rank-block count is a template parameter (r_k rounded up to a
//     multiple of 64), so the rebuild is straight-line code the compiler can software-pipeline.
//   * The waves walk the 32-position blocks in lockstep. Each block's K latent (32 x r_k, tiled layout)
//     is staged once in LDS (every wave loads an eighth, two register sets deep), two blocks ahead of
//     use; every wave rebuilds its 16 dims of K^T for the block on MFMA (v_mfma_f32_16x16x32_bf16),
//     rotates them in-lane (block-relative RoPE, this wave's part of the table held in registers; the
//     query is rotated back by the block base) and contracts them with its 16 dims of the query
//     (v_mfma_f32_16x16x16_bf16), giving a partial score tile.
//   * The eight partial tiles go through LDS (double-buffered by block parity); after the block's
//     barrier every wave sums them and runs the same online softmax and latent-space PV for the block,
//     then rebuilds the next block's scores in the same barrier interval, so the LDS and exp latencies
//     of one block overlap the rebuild MFMAs of the next and each block needs a single barrier.
//   * V stays in latent space: wave w owns an eighth of the V latent tiles and accumulates
//     O_lat^T = V_lat^T P^T for them; the V tiles come straight from HBM two blocks ahead. The per-head
//     V rebuild is applied once at the end, out = O_lat u_v[h] / l, in fp32, which is the same sum as
//     softmax(q K^T) (V_lat u_v[h]) without materialising V.
//   * Workgroups of the heads that share a latent are numbered so they land on the same XCD (the
//     dispatcher deals consecutive workgroup ids round-robin over the 8 XCDs): their latent reads then
//     meet in that XCD's L2 instead of each going to HBM.
#include "palu_kernel.h"

namespace {

constexpr int G_NW = 8;                 // waves per workgroup; wave w owns head dims 16w .. 16w + 15
constexpr int G_MAXKB = 16;             // r_k <= 512: 32-wide rank blocks of the K latent
constexpr int G_MAXTPW = 4;             // r_v <= 512: 16-wide V tiles per wave
constexpr int G_LAT_TILES = 2 * G_MAXKB;              // 1 KB tiles of one staged K-latent block

typedef short s16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma16k16(bf16x4 a, bf16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                   0, 0, 0);
}

__device__ __forceinline__ bf16x4 pack4(f32x4 x) {
  bf16x4 r;
  r[0] = (__bf16)x[0]; r[1] = (__bf16)x[1]; r[2] = (__bf16)x[2]; r[3] = (__bf16)x[3];
  return r;
}

// LDS map:
//   lat   two staged K-latent blocks, K-tile order, [buffer][tile][lane] bf16x8        64 KB
//   pbuf  partial scores, [block parity][wave][tile c][lane] float4                    32 KB
//   tl    (cos, sin) of angle 32*Lo*f, Lo < 32                                          16 KB
//   qs    the item's query rows (zero rows past rep)                                     4 KB
//   th    (cos, sin) of angle 1024*H*f, H < ceil(S / 1024)                        S/1024 x 512 B
//   kc    staging of cs_tab rows 0..31 in the prologue, overlaying pbuf; the epilogue's O_lat
//         [16 heads][r_v + 4] fp32 and final (m, l) per head overlay lat, its reduction buffer pbuf.
struct GSmem {
  static constexpr int LAT = 0;
  static constexpr int PBUF = LAT + 2 * G_LAT_TILES * 1024;
  static constexpr int TL = PBUF + 2 * G_NW * 2 * 64 * 16;
  static constexpr int QS = TL + 32 * 64 * 8;
  static constexpr int TH = QS + 16 * HD * 2;
  static constexpr int OLAT_STRIDE = 512 + 4;
  static constexpr int ML = LAT + 16 * OLAT_STRIDE * 4;
  static_assert(ML + 16 * 2 * 4 <= PBUF, "the epilogue buffers overlay the latent stage");
  static_assert(32 * 64 * 8 <= TL - PBUF, "the cs_tab staging rows overlay pbuf");
  static_assert(G_NW * 64 * 8 * 4 <= TL - PBUF, "the epilogue reduction overlays pbuf");
  __host__ __device__ static int bytes(int S) { return TH + ((S + 1023) / 1024) * 64 * 8; }
};

// KBC: rank blocks of 32 the rebuild runs (r_k / 32 rounded up to even, at most 16).
template <int KBC, typename TabT, typename OutT>
__global__ __launch_bounds__(G_NW * 64) void palu_glrd_kernel(const DecodeArgs a, int n_streams) {
  static_assert(KBC % 2 == 0 && KBC >= 2 && KBC <= G_MAXKB, "rank-block count");
  constexpr int LPW = (2 * KBC + G_NW - 1) / G_NW;      // K-latent tiles each wave stages per block
  extern __shared__ __attribute__((aligned(16))) char smem[];
  char* lat = smem + GSmem::LAT;
  float2* tl = reinterpret_cast<float2*>(smem + GSmem::TL);
  float2* th = reinterpret_cast<float2*>(smem + GSmem::TH);
  float2* kc = reinterpret_cast<float2*>(smem + GSmem::PBUF);
  __bf16* qs_lds = reinterpret_cast<__bf16*>(smem + GSmem::QS);
  float4* pbuf = reinterpret_cast<float4*>(smem + GSmem::PBUF);

  // Workgroup id -> (latent stream, head in group): ids 8*q + x with the same x share an XCD, and the
  // heads of one stream get consecutive q, so they share x.
  const int L = blockIdx.x;
  const int x8 = L & 7, q8 = L >> 3;
  const int hig = q8 % a.hpg;
  const int sigma = (q8 / a.hpg) * 8 + x8;
  if (sigma >= n_streams) return;                       // padding workgroup (uniform: whole group exits)
  const int n_groups = a.n_kv / a.hpg;
  const int split = sigma % a.n_splits;
  const int bg = sigma / a.n_splits;
  const int b = bg / n_groups, grp = bg - b * n_groups;
  const int kvh = grp * a.hpg + hig;
  const int item = b * a.n_kv + kvh;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int KB = a.rk >> 5;                             // rank blocks of the K latent (KBC - 1 or KBC)
  const int NT = 2 * KB;                                // 1 KB tiles per K-latent block
  const int VT = a.rv >> 4;                             // 16-wide V tiles
  const int TPW = (VT + G_NW - 1) / G_NW;               // V tiles per wave

  int len = a.cur_pos[b] + 1;
  len = len < 0 ? 0 : (len > a.S ? a.S : len);
  const int s_lo = split * a.split_len;
  const int s_hi = min(len, s_lo + a.split_len);
  const int nblk = s_hi > s_lo ? (s_hi - s_lo + BLK - 1) / BLK : 0;

  const __bf16* kbase = a.k + b * a.k_sb + grp * a.k_sg;
  const __bf16* vbase = a.v + b * a.v_sb + grp * a.v_sg;

  // ---- prologue: tables, query rows, this wave's u_k^T slice ----------------------------------------
  {
    const TabT* cs = static_cast<const TabT*>(a.cs);
    const int n_hi = (a.S + 1023) / 1024;
    const int n_rows = 64 + n_hi;                        // 32 K rows, 32 low-base rows, n_hi high-base rows
    constexpr int RPW = (64 + 64 + G_NW - 1) / G_NW;
    float4 rowv[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int r = w + i * G_NW;
      int t = r < 32 ? r : (r < 64 ? 32 * (r - 32) : 1024 * (r - 64));
      t = (r < n_rows && t < a.cs_rows) ? t : 0;
      rowv[i] = load4f(cs + (long long)t * (2 * HD) + 4 * lane);
    }
    if (tid < 256) {
      const int qh = tid >> 4, qc = (tid & 15) * 8;    // 16 rows x 16 pieces of 8
      bf16x8 qrow = bf16x8{};
      if (qh < a.rep)
        qrow = *reinterpret_cast<const bf16x8*>(a.q + ((long long)b * a.n_q + (long long)kvh * a.rep + qh) * HD + qc);
      *reinterpret_cast<bf16x8*>(qs_lds + qh * HD + qc) = qrow;
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int r = w + i * G_NW;
      if (r < n_rows) {
        const int t = r < 32 ? r : (r < 64 ? 32 * (r - 32) : 1024 * (r - 64));
        const bool ok = t < a.cs_rows;
        float2* dst = r < 32 ? kc + r * 64 : (r < 64 ? tl + (r - 32) * 64 : th + (r - 64) * 64);
        float* d0 = reinterpret_cast<float*>(dst + 2 * (lane & 31)) + (lane >> 5);
        d0[0] = ok ? rowv[i].x : (lane < 32 ? 1.f : 0.f);
        d0[2] = ok ? rowv[i].z : (lane < 32 ? 1.f : 0.f);
      }
    }
  }

  // u_k^T slice: A operand of the rebuild, row d = 16w + n, ranks 32kb + 8g .. +7 (zero past r_k).
  bf16x8 ukA[KBC];
  {
    const __bf16* ukp = a.w_rot + (long long)kvh * a.rk * (2 * HD) + 16 * w + n;
#pragma unroll
    for (int kb = 0; kb < KBC; ++kb) {
      bf16x8 v = bf16x8{};
      if (kb < KB) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = ukp[(long long)(32 * kb + 8 * g + j) * (2 * HD)];
      }
      ukA[kb] = v;
    }
  }

  // Loads of one block: this wave's K-latent tiles (tile w + 8i) and its V tiles (tile w * TPW + i).
  // They are ordinary (cached) loads: the heads of a group read the same latent rows at about the same
  // time, and the L2 serves all but the first. Past the last block (or past the tile count) the same
  // instructions read the first tile of block 0 of the split, so every path issues the same loads and
  // stores; that data is never used.
  auto load_lat = [&](int j, bf16x8 (&la)[LPW]) {
    const bool live = j < nblk;
    const __bf16* kb0 = kbase + (live ? (long long)((s_lo >> 5) + j) * (32 * a.rk) : (long long)(s_lo >> 5) * (32 * a.rk)) + lane * 8;
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int t = w + G_NW * i;
      la[i] = *reinterpret_cast<const bf16x8*>(kb0 + (t < NT ? t : 0) * 512);
    }
  };
  auto store_lat = [&](int buf, const bf16x8 (&la)[LPW]) {
    bf16x8* dst = reinterpret_cast<bf16x8*>(lat + buf * (G_LAT_TILES * 1024));
#pragma unroll
    for (int i = 0; i < LPW; ++i) dst[(w + G_NW * i) * 64 + lane] = la[i];
  };
  auto load_v = [&](int j, bf16x8 (&va)[G_MAXTPW]) {
    const bool live = j < nblk;
    const __bf16* vb0 = vbase + (live ? (long long)((s_lo >> 5) + j) * (32 * a.rv) : (long long)(s_lo >> 5) * (32 * a.rv)) + lane * 8;
#pragma unroll
    for (int i = 0; i < G_MAXTPW; ++i) {
      const int mt = w * TPW + i;
      va[i] = *reinterpret_cast<const bf16x8*>(vb0 + ((i < TPW && mt < VT) ? mt : 0) * 512);
    }
  };

  // Query rotated back by the block base and scaled by scale * log2 e, this wave's 16 dims: lane
  // (head n, g) holds dims 16w + 4g .. +3 (frequency pairs 8w + 2g, +1), the B operand of the QK MFMA.
  auto make_q = [&](int base) -> bf16x4 {
    const int J = base >> 5;
    const int f0 = 8 * w + 2 * g;
    const float4 lo = *reinterpret_cast<const float4*>(tl + (J & 31) * 64 + f0);
    const float4 hi = *reinterpret_cast<const float4*>(th + (J >> 5) * 64 + f0);
    const bf16x4 qv = *reinterpret_cast<const bf16x4*>(qs_lds + n * HD + 16 * w + 4 * g);
    const float lc[2] = {lo.x, lo.z}, ls[2] = {lo.y, lo.w}, hc[2] = {hi.x, hi.z}, hs[2] = {hi.y, hi.w};
    bf16x4 r;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const float cf = (hc[p] * lc[p] - hs[p] * ls[p]) * a.qscale;
      const float sf = (hs[p] * lc[p] + hc[p] * ls[p]) * a.qscale;
      const float x0 = (float)qv[2 * p], x1 = (float)qv[2 * p + 1];
      r[2 * p] = (__bf16)(x0 * cf + x1 * sf);                        // R_{-base}
      r[2 * p + 1] = (__bf16)(x1 * cf - x0 * sf);
    }
    return r;
  };

  f32x4 O[G_MAXTPW];
#pragma unroll
  for (int i = 0; i < G_MAXTPW; ++i) O[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = NEG_INF, l_run = 0.f;
  float4 rot[2];                                         // this wave's rotation of block offsets, tile c

  // Partial scores of block j: rebuild this wave's K^T slice from lat buffer j & 1, rotate, contract
  // with this wave's query dims, store the tile in pbuf[j & 1]. Rank blocks past r_k multiply a zero
  // u_k slice with a tile of the same position order, so they add exact zeros.
  auto scores = [&](int j) __attribute__((always_inline)) {
    const bf16x4 qB = make_q(s_lo + j * BLK);
    const bf16x8* lt = reinterpret_cast<const bf16x8*>(lat + (j & 1) * (G_LAT_TILES * 1024));
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int kb = 0; kb < KBC; ++kb) {
      const int kbr = kb < KB ? kb : 0;
#pragma unroll
      for (int c = 0; c < 2; ++c) acc[c] = mfma16(ukA[kb], lt[(c * KB + kbr) * 64 + lane], acc[c]);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const float4 t = rot[c];
      const float x0 = acc[c][0], x1 = acc[c][1], x2 = acc[c][2], x3 = acc[c][3];
      acc[c][0] = x0 * t.x - x1 * t.y;
      acc[c][1] = x1 * t.x + x0 * t.y;
      acc[c][2] = x2 * t.z - x3 * t.w;
      acc[c][3] = x3 * t.z + x2 * t.w;
      const f32x4 sc = mfma16k16(pack4(acc[c]), qB, f32x4{0.f, 0.f, 0.f, 0.f});
      pbuf[(((j & 1) * G_NW + w) * 2 + c) * 64 + lane] = make_float4(sc[0], sc[1], sc[2], sc[3]);
    }
  };

  // Online softmax and latent-space PV of block j, once every wave's partial tile of the block is in
  // pbuf[j & 1]. The lazy rescale and the PV over the wave's tiles are branch-free (a tile past r_v
  // multiplies a dummy V tile into an accumulator that is never stored), so the whole barrier
  // interval is one basic block the compiler can interleave with the next block's rebuild.
  auto softmax_pv = [&](auto partial_tag, int j, const bf16x8 (&va)[G_MAXTPW]) __attribute__((always_inline)) {
    constexpr bool partial = decltype(partial_tag)::value;
    const int base = s_lo + j * BLK;
    f32x4 sc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int ww = 0; ww < G_NW; ++ww) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const float4 v = pbuf[(((j & 1) * G_NW + ww) * 2 + c) * 64 + lane];
        sc[c] += f32x4{v.x, v.y, v.z, v.w};
      }
    }
    if constexpr (partial) {
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (base + 8 * g + 4 * c + i >= s_hi) sc[c][i] = NEG_INF;
    }
    float bm = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                     fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
    bm = wave_max_xor48(bm);
    const bool need = __any(bm > m_run + LAZY_RESCALE_LOG2);
    const float mn = need ? fmaxf(m_run, bm) : m_run;
    const float alpha = need ? ((m_run == NEG_INF) ? 0.f : __builtin_amdgcn_exp2f(m_run - mn)) : 1.f;
#pragma unroll
    for (int i = 0; i < G_MAXTPW; ++i) O[i] *= alpha;
    l_run *= alpha;
    m_run = mn;
    const float mref = (m_run == NEG_INF) ? 0.f : m_run;
    f32x4 p[2];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) p[c][i] = __builtin_amdgcn_exp2f(sc[c][i] - mref);
    l_run += (p[0][0] + p[0][1]) + (p[0][2] + p[0][3]) + (p[1][0] + p[1][1]) + (p[1][2] + p[1][3]);
    const bf16x8 pB = pack8(p[0], p[1]);
#pragma unroll
    for (int i = 0; i < G_MAXTPW; ++i) {
      bf16x8 vA = va[i];
      if constexpr (partial) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (base + 8 * g + e >= s_hi) vA[e] = (__bf16)0.0f;
      }
      O[i] = mfma16(vA, pB, O[i]);
    }
  };

  // Pipeline. Between two barriers, step j: write block j + 2 (register set j & 1, loaded in step
  // j - 1) into lat buffer j & 1, which scores(j) finished reading before the barrier; load block
  // j + 3 into the other set; softmax and PV of block j from its partial tiles; load V of block j + 2
  // into the V set block j used; scores(j + 1) from lat buffer (j + 1) & 1, staged in step j - 1.
  // The prologue stages blocks 0 and 1, loads block 2 into set 0 and V of blocks 0 and 1, and runs
  // scores(0). Steps run in pairs so every register set keeps a fixed role.
  const std::integral_constant<bool, false> full_blk;
  const std::integral_constant<bool, true> partial_blk;
  const int nfull = s_hi > s_lo ? (s_hi - s_lo) / BLK : 0;
  bf16x8 la0[LPW], la1[LPW], va0[G_MAXTPW], va1[G_MAXTPW];
  load_lat(0, la0);
  load_lat(1, la1);
  store_lat(0, la0);
  store_lat(1, la1);
  load_lat(2, la0);
  load_v(0, va0);
  load_v(1, va1);
  __syncthreads();                                      // kc, tl, th, qs, latent blocks 0 and 1
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int t = 8 * (n >> 2) + 4 * c + (n & 3);        // block offset of this lane's position
    const int f = 8 * w + 2 * g;                          // frequency pair of this lane's dims 0, 1
    const float2 x = kc[t * 64 + f], y = kc[t * 64 + f + 1];
    rot[c] = make_float4(x.x, x.y, y.x, y.y);
  }
  __syncthreads();                                      // kc (overlaying pbuf) read by every wave
  if (nblk > 0) scores(0);
  __syncthreads();

  // LS: set holding block j + 2 (written to LDS), LL: set receiving block j + 3, VC: V set of block j,
  // then receiving V of block j + 2.
  auto step = [&](int j, bf16x8 (&LS)[LPW], bf16x8 (&LL)[LPW], bf16x8 (&VC)[G_MAXTPW]) __attribute__((always_inline)) {
    store_lat(j & 1, LS);
    load_lat(j + 3, LL);
    softmax_pv(full_blk, j, VC);
    load_v(j + 2, VC);
    scores(j + 1);
    __syncthreads();
  };
  int j = 0;
  for (; j + 2 < nfull; j += 2) {
    step(j, la0, la1, va0);
    step(j + 1, la1, la0, va1);
  }
  if (j + 1 < nfull) {
    step(j, la0, la1, va0);
    ++j;
  }
  // j == nfull - 1 when nfull > 0: the last full block's partial tiles are in pbuf
  if (nfull > 0) {
    if (j & 1) softmax_pv(full_blk, j, va1);
    else softmax_pv(full_blk, j, va0);
  }
  if (nfull < nblk) {
    // partial last block nfull: latent staged in buffer nfull & 1 (scores(0) already ran when nfull == 0),
    // V in set nfull & 1
    if (nfull > 0) scores(nfull);
    __syncthreads();
    if (nfull & 1) softmax_pv(partial_blk, nfull, va1);
    else softmax_pv(partial_blk, nfull, va0);
  }

  // ---- epilogue: out = O_lat u_v[h] / l -----------------------------------------------------------
  l_run = wave_sum_xor48(l_run);
  float* olat = reinterpret_cast<float*>(smem + GSmem::LAT);
  float* ml = reinterpret_cast<float*>(smem + GSmem::ML);
  __syncthreads();                                      // every wave is past its last latent store
  // lanes (n, g) hold O^T[16 mt + 4 g + i][head n]
#pragma unroll
  for (int i = 0; i < G_MAXTPW; ++i) {
    const int mt = w * TPW + i;
    if (i < TPW && mt < VT) {
#pragma unroll
      for (int e = 0; e < 4; ++e) olat[n * GSmem::OLAT_STRIDE + 16 * mt + 4 * g + e] = O[i][e];
    }
  }
  if (w == 0 && lane < 16) { ml[2 * lane] = m_run; ml[2 * lane + 1] = l_run; }
  __syncthreads();
  // Thread (unit u = (head, 8 output dims), part) sums its share of the r_v ranks; the parts of a
  // unit are added through LDS (pbuf).
  const __bf16* uv = a.u_v + (long long)kvh * a.rv * HD;
  const int units = a.rep * (HD / 8);
  const int parts = (G_NW * 64) / units;
  const int per = (a.rv + parts - 1) / parts;
  float* red = reinterpret_cast<float*>(pbuf);
  if (tid < units * parts) {
    const int u = tid % units, part = tid / units;
    const int h = u / (HD / 8), d8 = (u % (HD / 8)) * 8;
    const float* orow = olat + h * GSmem::OLAT_STRIDE;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const int r0 = part * per, r1 = min(a.rv, r0 + per);
    for (int r = r0; r < r1; ++r) {
      const bf16x8 uvv = *reinterpret_cast<const bf16x8*>(uv + (long long)r * HD + d8);
      const float o = orow[r];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += o * (float)uvv[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) red[(part * units + u) * 8 + e] = acc[e];
  }
  __syncthreads();
  if (tid < units) {
    const int u = tid, h = u / (HD / 8), d8 = (u % (HD / 8)) * 8;
    const float M = ml[2 * h], Lsum = ml[2 * h + 1];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = 0.f;
      for (int part = 0; part < parts; ++part) acc += red[(part * units + u) * 8 + e];
      if (a.n_splits == 1) {
        OutT* o = static_cast<OutT*>(a.out) + ((long long)b * a.n_q + (long long)kvh * a.rep + h) * HD + d8 + e;
        store_out(o, Lsum > 0.f ? acc / Lsum : 0.f);
      } else {
        float* wrow = a.ws + (((long long)item * a.n_splits + split) * 16 + h) * (HD + 2);
        wrow[d8 + e] = acc;
        if (d8 + e == 0) { wrow[HD] = M; wrow[HD + 1] = Lsum; }
      }
    }
  }
}

template <int KBC, typename TabT, typename OutT>
int launch_glrd(const DecodeArgs& a0, hipStream_t stream) {
  DecodeArgs a = a0;
  const int items = a.B * a.n_kv;
  const Plan p = plan_splits(items, a.S, G_NW);
  a.split_len = p.split_len;
  a.n_splits = p.n_splits;
  const size_t need = ws_bytes(items, p.n_splits, HD);
  if (need > 0 && (a.ws == nullptr || a.ws_bytes < need))
    return fail(PALU_EINVAL, "workspace of %zu bytes needed (palu_decode_workspace_bytes), got %zu", need, a.ws_bytes);
  const int n_groups = a.n_kv / a.hpg;
  const int n_streams = a.B * n_groups * a.n_splits;
  const long long n_wg = (long long)((n_streams + 7) / 8) * 8 * a.hpg;
  if (n_wg > 0x7fffffff) return fail(PALU_EUNSUPPORTED, "grouped-latent grid of %lld workgroups", n_wg);
  auto kern = palu_glrd_kernel<KBC, TabT, OutT>;
  const int lds = GSmem::bytes(a.S);
  if (lds > 160 * 1024) return fail(PALU_EUNSUPPORTED, "seq_len %d needs %d bytes of LDS (max 163840)", a.S, lds);
  static int attr_set = 0;
  if (attr_set < lds) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return fail(PALU_EHIP, "hipFuncSetAttribute: %s", hipGetErrorString(e));
    attr_set = lds;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)n_wg), dim3(G_NW * 64), lds, stream, a, n_streams);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PALU_EHIP, "grouped-latent decode kernel launch: %s", hipGetErrorString(e));
  if (a.n_splits > 1) {
    hipLaunchKernelGGL((palu_merge_kernel<HD, OutT>), dim3(items), dim3(256), 0, stream, a.ws, a.out, a.n_splits,
                       a.rep, a.n_q, a.n_kv);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(PALU_EHIP, "merge kernel launch: %s", hipGetErrorString(e));
  }
  return PALU_OK;
}

template <typename TabT, typename OutT>
int launch_glrd_kb(const DecodeArgs& a, hipStream_t s) {
  switch ((a.rk / 32 + 1) / 2) {               // rank blocks rounded up to even, in pairs
    case 1: return launch_glrd<2, TabT, OutT>(a, s);
    case 2: return launch_glrd<4, TabT, OutT>(a, s);
    case 3: return launch_glrd<6, TabT, OutT>(a, s);
    case 4: return launch_glrd<8, TabT, OutT>(a, s);
    case 5: return launch_glrd<10, TabT, OutT>(a, s);
    case 6: return launch_glrd<12, TabT, OutT>(a, s);
    case 7: return launch_glrd<14, TabT, OutT>(a, s);
    case 8: return launch_glrd<16, TabT, OutT>(a, s);
  }
  return fail(PALU_EUNSUPPORTED, "grouped-latent r_k %d (32 .. 512 in steps of 32)", a.rk);
}

}  // namespace

namespace palu {

int dispatch_glrd(const DecodeArgs& a, int cs_dtype, int out_dtype, hipStream_t s) {
  const bool f32o = out_dtype == PALU_DTYPE_F32;
  if (cs_dtype == PALU_DTYPE_F32) return f32o ? launch_glrd_kb<float, float>(a, s) : launch_glrd_kb<float, __bf16>(a, s);
  return f32o ? launch_glrd_kb<__bf16, float>(a, s) : launch_glrd_kb<__bf16, __bf16>(a, s);
}

}  // namespace palu
