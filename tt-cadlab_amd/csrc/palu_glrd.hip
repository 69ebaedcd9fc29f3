// Fused decode over grouped latents with V rebuilt in-kernel (G-LRD): heads_per_group KV heads share
// one K latent and one V latent of rank up to 512, and every KV head has its own 128-column slices of
// U_k and U_v (palu_sdpa_decode with u_v; docs/superpowers/specs/2026-09-12-palu-tt-stage2b-design.md:
// 120-142, fp32 model palu_tt/fused.py:82-107 with u_v).
//
// Shape of the kernel (one workgroup = one (row, KV head) item and one sequence split, 4 waves):
//   * The 4 waves split the head dim: wave w owns dims 32w .. 32w+31, and keeps that 32 x r_k slice of
//     u_k^T in registers for the whole kernel, so U_k is read once per workgroup, whatever r_k.
//   * The waves walk the 32-position blocks in lockstep. Each block's K latent (32 x r_k, tiled layout)
//     is staged once in LDS (every wave loads a quarter), two blocks ahead of use; every wave rebuilds
//     its 32 dims of K^T for the block on MFMA, rotates them (block-relative RoPE table in LDS, query
//     rotated back by the block base) and contracts them with its slice of the query. The four partial
//     scores are summed through LDS, so every wave holds the full scores and runs the same online
//     softmax.
//   * V stays in latent space: wave w owns a quarter of the V latent columns and accumulates
//     O_lat^T = V_lat^T P^T for them; the V tiles come straight from HBM one block ahead. The per-head
//     V rebuild is applied once at the end, out = O_lat u_v[h] / l, in fp32, which is the same sum as
//     softmax(q K^T) (V_lat u_v[h]) without materialising V.
//   * Workgroups of the heads that share a latent are numbered so they land on the same XCD (the
//     dispatcher deals consecutive workgroup ids round-robin over the 8 XCDs): their latent reads then
//     meet in that XCD's L2 instead of each going to HBM.
#include "palu_kernel.h"

namespace {

constexpr int G_NW = 4;                 // waves per workgroup; wave w owns head dims 32w .. 32w + 31
constexpr int G_MAXKB = 16;             // r_k <= 512: 32-wide rank blocks of the K latent
constexpr int G_MAXTPW = 8;             // r_v <= 512: 16-wide V tiles per wave
constexpr int G_LAT_TILES = 2 * G_MAXKB;              // 1 KB tiles of one staged K-latent block
constexpr int G_LAT_PER_WAVE = G_LAT_TILES / G_NW;    // tiles each wave loads per block

// LDS map:
//   rtab  block-relative K rotation in lane order [tile c][row tile][lane] float4       16 KB
//   lat   two staged K-latent blocks, K-tile order, [buffer][tile][lane] bf16x8        64 KB
//   qx    per wave, the rotated query regrouped into MFMA operand order                  16 KB
//   tl    (cos, sin) of angle 32*Lo*f, Lo < 32                                           16 KB
//   qs    the item's query rows                                                           4 KB
//   sbuf  per wave, its partial scores [wave][tile c][lane] float4                         8 KB
//   th    (cos, sin) of angle 1024*H*f, H < ceil(S / 1024)                          S/1024 x 512 B
//   kc    staging of cs_tab rows 0..31 while rtab is built (overlays qx); olat, the epilogue's
//         O_lat [16 heads][r_v + 4] fp32, and the final (m, l) per head overlay lat.
struct GSmem {
  static constexpr int RTAB = 0;
  static constexpr int LAT = RTAB + 2 * 8 * 64 * 16;
  static constexpr int QX = LAT + 2 * G_LAT_TILES * 1024;
  static constexpr int TL = QX + G_NW * 4096;
  static constexpr int QS = TL + 32 * 64 * 8;
  static constexpr int SBUF = QS + 16 * HD * 2;
  static constexpr int TH = SBUF + G_NW * 2 * 64 * 16;
  static constexpr int OLAT_STRIDE = 512 + 4;
  static constexpr int ML = LAT + 16 * OLAT_STRIDE * 4;
  static_assert(ML + 16 * 2 * 4 <= QX, "the epilogue buffers overlay the latent stage");
  __host__ __device__ static int bytes(int S) { return TH + ((S + 1023) / 1024) * 64 * 8; }
};

template <typename TabT, typename OutT>
__global__ __launch_bounds__(G_NW * 64) void palu_glrd_kernel(const DecodeArgs a, int n_streams) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  float4* rtab = reinterpret_cast<float4*>(smem + GSmem::RTAB);
  char* lat = smem + GSmem::LAT;
  float2* tl = reinterpret_cast<float2*>(smem + GSmem::TL);
  float2* th = reinterpret_cast<float2*>(smem + GSmem::TH);
  float2* kc = reinterpret_cast<float2*>(smem + GSmem::QX);
  __bf16* qs_lds = reinterpret_cast<__bf16*>(smem + GSmem::QS);
  float4* sbuf = reinterpret_cast<float4*>(smem + GSmem::SBUF);

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
  __bf16* qx = reinterpret_cast<__bf16*>(smem + GSmem::QX + w * 4096);
  const int KB = a.rk >> 5;                             // rank blocks of the K latent
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
    const int qh = tid >> 4, qc = (tid & 15) * 8;      // 16 rows x 16 pieces of 8
    bf16x8 qrow = bf16x8{};
    if (qh < a.rep)
      qrow = *reinterpret_cast<const bf16x8*>(a.q + ((long long)b * a.n_q + (long long)kvh * a.rep + qh) * HD + qc);
    *reinterpret_cast<bf16x8*>(qs_lds + qh * HD + qc) = qrow;
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
    __syncthreads();
    for (int e = tid; e < 2 * 8 * 64; e += G_NW * 64) {
      const int l = e & 63, rt = (e >> 6) & 7, c = e >> 9;
      const int nn = l & 15, gg = l >> 4;
      const int t = 8 * (nn >> 2) + 4 * c + (nn & 3);
      const int f = 8 * rt + 2 * gg;
      const float2 x = kc[t * 64 + f], y = kc[t * 64 + f + 1];
      rtab[e] = make_float4(x.x, x.y, y.x, y.y);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4096 / (64 * 16); ++i)
      reinterpret_cast<float4*>(qx)[i * 64 + lane] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  // u_k^T slice: A operand of the rebuild, row d = 32w + 16h + n, ranks 32kb + 8g .. +7.
  bf16x8 ukA[2][G_MAXKB];
  {
    const __bf16* ukp = a.w_rot + (long long)kvh * a.rk * (2 * HD);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int d = 32 * w + 16 * h + n;
#pragma unroll
      for (int kb = 0; kb < G_MAXKB; ++kb) {
        bf16x8 v = bf16x8{};
        if (kb < KB) {
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = ukp[(long long)(32 * kb + 8 * g + j) * (2 * HD) + d];
        }
        ukA[h][kb] = v;
      }
    }
  }

  // Loads of one block: this wave's quarter of the K-latent tiles (tile w + 4i) and its V tiles
  // (tile w * TPW + i). They are ordinary (cached) loads: the heads of a group read the same latent
  // rows at about the same time, and the L2 serves all but the first. Past the last block (or past the tile count) the same instructions read the
  // first tiles of block 0 of the stream, so every path issues the same loads; that data is unused.
  auto load_lat = [&](int j, bf16x8 (&la)[G_LAT_PER_WAVE]) {
    const bool live = j < nblk;
    const __bf16* kb0 = kbase + (live ? (long long)((s_lo >> 5) + j) * (32 * a.rk) : 0) + lane * 8;
#pragma unroll
    for (int i = 0; i < G_LAT_PER_WAVE; ++i) {
      const int t = w + G_NW * i;
      la[i] = *reinterpret_cast<const bf16x8*>(kb0 + (t < NT ? t : 0) * 512);
    }
  };
  auto store_lat = [&](int buf, const bf16x8 (&la)[G_LAT_PER_WAVE]) {
    bf16x8* dst = reinterpret_cast<bf16x8*>(lat + buf * (G_LAT_TILES * 1024));
#pragma unroll
    for (int i = 0; i < G_LAT_PER_WAVE; ++i) {
      const int t = w + G_NW * i;
      if (t < NT) dst[t * 64 + lane] = la[i];
    }
  };
  auto load_v = [&](int j, bf16x8 (&va)[G_MAXTPW]) {
    const bool live = j < nblk;
    const __bf16* vb0 = vbase + (live ? (long long)((s_lo >> 5) + j) * (32 * a.rv) : 0) + lane * 8;
#pragma unroll
    for (int i = 0; i < G_MAXTPW; ++i) {
      const int mt = w * TPW + i;
      va[i] = *reinterpret_cast<const bf16x8*>(vb0 + ((i < TPW && mt < VT) ? mt : 0) * 512);
    }
  };

  // Query rotated back by the block base, scaled by scale * log2 e, for this wave's 32 dims only:
  // lane (head l/4, dims 32w + 8(l%4) .. +7, i.e. frequency pairs 16w + 4(l%4) .. +3), regrouped
  // through the wave's LDS area into the QK operand order d(j) = 16*(2w + j/4) + 4*g + j%4.
  bf16x8 qB;
  auto make_q = [&](int base) {
    const int J = base >> 5;
    const int hq = lane >> 2, qd = lane & 3;
    const int qf = 4 * w + qd;                       // 8-dim group of the head dim
    const float4* lo4 = reinterpret_cast<const float4*>(tl + (J & 31) * 64 + 4 * qf);
    const float4* hi4 = reinterpret_cast<const float4*>(th + (J >> 5) * 64 + 4 * qf);
    const float4 l01 = lo4[0], l23 = lo4[1], h01 = hi4[0], h23 = hi4[1];
    const float lc[4] = {l01.x, l01.z, l23.x, l23.z}, ls[4] = {l01.y, l01.w, l23.y, l23.w};
    const float hc[4] = {h01.x, h01.z, h23.x, h23.z}, hs[4] = {h01.y, h01.w, h23.y, h23.w};
    const int rt = qf >> 1, g0 = 2 * (qf & 1);
    if (hq < a.rep) {
      const bf16x8 qv = *reinterpret_cast<const bf16x8*>(qs_lds + hq * HD + 8 * qf);
      bf16x4 y0, y1;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const float cf = (hc[p] * lc[p] - hs[p] * ls[p]) * a.qscale;
        const float sf = (hs[p] * lc[p] + hc[p] * ls[p]) * a.qscale;
        const float x0 = (float)qv[2 * p], x1 = (float)qv[2 * p + 1];
        const float r0 = x0 * cf + x1 * sf, r1 = x1 * cf - x0 * sf;      // R_{-base}
        if (p < 2) { y0[2 * p] = (__bf16)r0; y0[2 * p + 1] = (__bf16)r1; }
        else { y1[2 * p - 4] = (__bf16)r0; y1[2 * p - 3] = (__bf16)r1; }
      }
      *reinterpret_cast<bf16x4*>(qx + ((hq * 4 + g0) * 8 + rt) * 4) = y0;
      *reinterpret_cast<bf16x4*>(qx + ((hq * 4 + g0 + 1) * 8 + rt) * 4) = y1;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    qB = *reinterpret_cast<const bf16x8*>(qx + ((n * 4 + g) * 8 + 2 * w) * 4);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  };

  f32x4 O[G_MAXTPW];
#pragma unroll
  for (int i = 0; i < G_MAXTPW; ++i) O[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = NEG_INF, l_run = 0.f;

  // One block, all waves together: rebuild this wave's K^T slice from the staged latent, rotate,
  // partial QK, exchange, online softmax, latent-space PV on this wave's V tiles.
  auto step = [&](auto partial_tag, int j, int buf, const bf16x8 (&va)[G_MAXTPW]) __attribute__((always_inline)) {
    constexpr bool partial = decltype(partial_tag)::value;
    const int base = s_lo + j * BLK;
    make_q(base);
    const bf16x8* lt = reinterpret_cast<const bf16x8*>(lat + buf * (G_LAT_TILES * 1024));
    f32x4 acc[2][2];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int h = 0; h < 2; ++h) acc[c][h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < G_MAXKB; ++kb) {
      if (kb < KB) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const bf16x8 lk = lt[(c * KB + kb) * 64 + lane];
#pragma unroll
          for (int h = 0; h < 2; ++h) acc[c][h] = mfma16(ukA[h][kb], lk, acc[c][h]);
        }
      }
    }
    f32x4 sc[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float4 t = rtab[(c * 8 + 2 * w + h) * 64 + lane];
        const float x0 = acc[c][h][0], x1 = acc[c][h][1], x2 = acc[c][h][2], x3 = acc[c][h][3];
        acc[c][h][0] = x0 * t.x - x1 * t.y;
        acc[c][h][1] = x1 * t.x + x0 * t.y;
        acc[c][h][2] = x2 * t.z - x3 * t.w;
        acc[c][h][3] = x3 * t.z + x2 * t.w;
      }
      sc[c] = mfma16(pack8(acc[c][0], acc[c][1]), qB, f32x4{0.f, 0.f, 0.f, 0.f});
      sbuf[(w * 2 + c) * 64 + lane] = make_float4(sc[c][0], sc[c][1], sc[c][2], sc[c][3]);
    }
    __syncthreads();                                     // partial scores of all waves are in sbuf
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ww = 0; ww < G_NW; ++ww) {
        const float4 v = sbuf[(ww * 2 + c) * 64 + lane];
        s[0] += v.x; s[1] += v.y; s[2] += v.z; s[3] += v.w;
      }
      sc[c] = s;
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
    if (__any(bm > m_run + LAZY_RESCALE_LOG2)) {
      const float mn = fmaxf(m_run, bm);
      const float alpha = (m_run == NEG_INF) ? 0.f : __builtin_amdgcn_exp2f(m_run - mn);
#pragma unroll
      for (int i = 0; i < G_MAXTPW; ++i) O[i] *= alpha;
      l_run *= alpha;
      m_run = mn;
    }
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
      if (i < TPW && w * TPW + i < VT) {
        bf16x8 vA = va[i];
        if constexpr (partial) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (base + 8 * g + e >= s_hi) vA[e] = (__bf16)0.0f;
        }
        O[i] = mfma16(vA, pB, O[i]);
      }
    }
  };

  // Pipeline: block j's latent is in lat buffer j & 1 when step j starts; its registers were loaded
  // two steps earlier. V of block j is loaded one step earlier. Two steps per trip keep the register
  // buffers in fixed roles.
  // Full blocks run in the pipelined loop; a partial last block (its latent staged by the pipeline)
  // runs once afterwards with masking, its V tiles loaded then.
  const std::integral_constant<bool, false> full_blk;
  const std::integral_constant<bool, true> partial_blk;
  const int nfull = s_hi > s_lo ? (s_hi - s_lo) / BLK : 0;
  bf16x8 la0[G_LAT_PER_WAVE], la1[G_LAT_PER_WAVE], va0[G_MAXTPW], va1[G_MAXTPW];
  load_lat(0, la0);
  load_v(0, va0);
  load_lat(1, la1);
  store_lat(0, la0);
  __syncthreads();
  for (int j = 0; j < nfull; j += 2) {
    load_lat(j + 2, la0);
    load_v(j + 1, va1);
    __builtin_amdgcn_sched_barrier(0);
    step(full_blk, j, 0, va0);
    store_lat(1, la1);
    __syncthreads();
    if (j + 1 < nfull) {
      load_lat(j + 3, la1);
      load_v(j + 2, va0);
      __builtin_amdgcn_sched_barrier(0);
      step(full_blk, j + 1, 1, va1);
      store_lat(0, la0);
      __syncthreads();
    }
  }
  if (nfull < nblk) {
    load_v(nfull, va0);
    step(partial_blk, nfull, nfull & 1, va0);
  }

  // ---- epilogue: out = O_lat u_v[h] / l -----------------------------------------------------------
  l_run = wave_sum_xor48(l_run);
  float* olat = reinterpret_cast<float*>(smem + GSmem::LAT);
  float* ml = reinterpret_cast<float*>(smem + GSmem::ML);
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
  // unit are added through LDS (sbuf).
  const __bf16* uv = a.u_v + (long long)kvh * a.rv * HD;
  const int units = a.rep * (HD / 8);
  const int parts = (G_NW * 64) / units;
  const int per = (a.rv + parts - 1) / parts;
  float* red = reinterpret_cast<float*>(sbuf);
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

template <typename TabT, typename OutT>
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
  auto kern = palu_glrd_kernel<TabT, OutT>;
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

}  // namespace

namespace palu {

int dispatch_glrd(const DecodeArgs& a, int cs_dtype, int out_dtype, hipStream_t s) {
  const bool f32o = out_dtype == PALU_DTYPE_F32;
  if (cs_dtype == PALU_DTYPE_F32) return f32o ? launch_glrd<float, float>(a, s) : launch_glrd<float, __bf16>(a, s);
  return f32o ? launch_glrd<__bf16, float>(a, s) : launch_glrd<__bf16, __bf16>(a, s);
}

}  // namespace palu
