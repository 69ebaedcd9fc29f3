// The scores pass of the grouped-latent decode (G-LRD pass 1; the other passes and the dispatch are in
// palu_glrd.hip). Two translation units instantiate it: palu_glrd.hip for K ranks above 256 and
// palu_glrd_narrow.hip for K ranks up to 256, which is built with the MFMA results in VGPRs (at those
// ranks the accumulators and the rest of the pair loop fit the 256 VGPRs, so the epilogue reads them
// without an accumulator-register copy each; at wider ranks that form spills and is slower).
#pragma once

#include "palu_kernel.h"

namespace {

// Lane K of the caller's row of 16 lanes, for every lane of the row (DPP row_newbcast:K).
template <int K>
__device__ __forceinline__ float row_bcast(float v) {
  static_assert(K >= 0 && K < 16, "row lane");
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x150 + K, 0xF, 0xF, false));
}

// f(std::integral_constant<int, I>) for I = B .. E - 1, unrolled at compile time.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

constexpr int G_QS = HD + 4;            // padded query row (fp32) of the scores kernel's LDS copy

// ---------------------------------------------------------------------------------------------------
// Pass 1: scores. One workgroup per (row, KV head, sequence split), 4 waves, one per SIMD, so each wave
// may hold up to 512 registers. The KV head's whole u_k^T (128 dims x r_k) sits in LDS as A tiles; each
// wave takes its own pairs of 32-position blocks and rebuilds K^T for all 128 dims x 64 positions at
// once (128 accumulator registers). A latent tile read from memory then feeds 8 MFMAs (one per 16-dim
// row tile) and a u_k^T tile read from LDS feeds 4 (one per 16-position tile). The pair-relative K
// rotation is the same for every pair, so it lives in registers as fp16 (cos, sin) pairs. Each query
// head's score is complete here; the PV pass reads one score per (head, position).
//
// LDS map (KBP = rank blocks rounded up to even), at most 154.3 KB (r_k 512) at every length:
//   ukt   u_k^T as A tiles [row tile 8][rank block KBP][lane] bf16x8 (zero past the group's r_k); at
//         least 32 KB,
//         because the prologue stages cs_tab rows 0..63 ([t][f] float2) in the same place
//   tl    (cos, sin) of angle 64*Lo*f, Lo < 16                                              8 KB
//   tm    (cos, sin) of angle 1024*Mi*f, Mi < 16                                            8 KB
//   tt    (cos, sin) of angle 16384*T*f, T < 4                                              2 KB
//   qs    the KV head's query rows times scale * log2 e, padded to G_QS               16 x G_QS fp32
// A pair base 64 J (J = 256 T + 16 Mi + Lo) takes its angle by two angle additions of these rows.
constexpr int G2_NW = 4;                // waves per workgroup of the scores kernel

template <int KBP>
struct G2Smem {
  static constexpr int UKT_BYTES = (8 * KBP * 1024 > 32768) ? 8 * KBP * 1024 : 32768;
  static constexpr int UKT = 0;
  static constexpr int TL = UKT + UKT_BYTES;
  static constexpr int TM = TL + 16 * 64 * 8;
  static constexpr int TT = TM + 16 * 64 * 8;
  static constexpr int QS = TT + 4 * 64 * 8;
  static constexpr int BYTES = QS + 16 * G_QS * 4;
  static_assert(BYTES <= 160 * 1024, "scores kernel LDS");
};

template <int KBP, typename TabT, bool ROWS>
__global__ __launch_bounds__(G2_NW * 64) void palu_glrd_scores_full_kernel(const DecodeArgs a, float* scores) {
  constexpr int R = (KBP % 4 == 0) ? 4 : 2;       // rank blocks of latent tiles in flight per wave
  using SM = G2Smem<KBP>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16x8* ukt = reinterpret_cast<bf16x8*>(smem + SM::UKT);
  float2* kc = reinterpret_cast<float2*>(smem + SM::UKT);
  float2* tl = reinterpret_cast<float2*>(smem + SM::TL);
  float2* tm = reinterpret_cast<float2*>(smem + SM::TM);
  float2* tt = reinterpret_cast<float2*>(smem + SM::TT);
  float* qs_lds = reinterpret_cast<float*>(smem + SM::QS);

  // Workgroup id -> (latent stream, KV head in group): ids 8*q + x with the same x share an XCD, and the
  // hpg workgroups of one stream (same row, group and split) get consecutive q, so they meet in one L2.
  // The launch covers groups grp_lo .. grp_lo + grp_cnt - 1, all of K rank rk_eff.
  const int n_groups = a.n_kv / a.hpg;
  const int L = blockIdx.x;
  const int x8 = L & 7, q8 = L >> 3;
  const int hig = q8 % a.hpg;
  const int sigma = (q8 / a.hpg) * 8 + x8;
  if (sigma >= a.B * a.grp_cnt * a.n_splits) return;  // padding workgroup (uniform)
  const int split = sigma % a.n_splits;
  const int bg = sigma / a.n_splits;
  const int b = bg / a.grp_cnt, grp = a.grp_lo + (bg - b * a.grp_cnt);
  const int kvh = grp * a.hpg + hig;
  const int QH = a.hpg * a.rep;
  const int NB = (a.S + BLK - 1) / BLK;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int KW = a.gkw[grp];                      // the group's stream width (row length of a ROWS cache)
  const int KB = KW >> 5;                         // rank blocks of the group's stream (tile addressing)
  const int KBe = a.rk_eff >> 5;                  // rank blocks of this group (the rest is never read)

  int len = a.cur_pos[b] + 1;
  len = len < 0 ? 0 : (len > a.S ? a.S : len);
  const int s_lo = split * a.split_len;
  const int s_hi = min(len, s_lo + a.split_len);
  const int nblk = s_hi > s_lo ? (s_hi - s_lo + BLK - 1) / BLK : 0;
  const int npairs = (nblk + 1) >> 1;
  const __bf16* kbase = a.k + b * a.k_sb + a.gko[grp];
  const int lrow = 8 * (n >> 2) + (n & 3);        // the lane's position in half-block 0 of a block

  // ---- prologue -----------------------------------------------------------------------------------
  // rot[cc][rt] = fp16 {cos f, sin f, cos f+1, sin f+1} at offset t = 32 hb + 8(n/4) + 4c + n%4 inside a
  // pair (cc = 2 hb + c), frequencies f = 8 rt + 2 g: the lane's accumulator dims 16 rt + 4 g .. +3.
  f16x4 rot[4][8];
  {
    const TabT* cs = static_cast<const TabT*>(a.cs);
    // rows: 64 K rows (t < 64), then 16 of 64 Lo, 16 of 1024 Mi, and ceil(S / 16384) of 16384 T
    const int n_rows = 96 + (a.S + 16383) / 16384;
    auto row_t = [](int r) { return r < 64 ? r : (r < 80 ? 64 * (r - 64) : (r < 96 ? 1024 * (r - 80) : 16384 * (r - 96))); };
    constexpr int RPW = (100 + G2_NW - 1) / G2_NW;
    float4 rowv[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int r = w + i * G2_NW;
      int t = row_t(r);
      t = (r < n_rows && t < a.cs_rows) ? t : 0;
      rowv[i] = load4f(cs + (long long)t * (2 * HD) + 4 * lane);
    }
    if (tid < 256) {
      const int qh = tid >> 4, qc = (tid & 15) * 8;    // 16 rows x 16 pieces of 8
      bf16x8 qrow = bf16x8{};
      if (qh < a.rep)
        qrow = *reinterpret_cast<const bf16x8*>(a.q + ((long long)b * a.n_q + (long long)kvh * a.rep + qh) * HD + qc);
      float4* qd = reinterpret_cast<float4*>(qs_lds + qh * G_QS + qc);
      qd[0] = make_float4((float)qrow[0] * a.qscale, (float)qrow[1] * a.qscale, (float)qrow[2] * a.qscale,
                          (float)qrow[3] * a.qscale);
      qd[1] = make_float4((float)qrow[4] * a.qscale, (float)qrow[5] * a.qscale, (float)qrow[6] * a.qscale,
                          (float)qrow[7] * a.qscale);
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int r = w + i * G2_NW;
      if (r < n_rows) {
        const int t = row_t(r);
        const bool ok = t < a.cs_rows;
        float2* dst = r < 64 ? kc + r * 64 : (r < 80 ? tl + (r - 64) * 64 : (r < 96 ? tm + (r - 80) * 64 : tt + (r - 96) * 64));
        float* d0 = reinterpret_cast<float*>(dst + 2 * (lane & 31)) + (lane >> 5);
        d0[0] = ok ? rowv[i].x : (lane < 32 ? 1.f : 0.f);
        d0[2] = ok ? rowv[i].z : (lane < 32 ? 1.f : 0.f);
      }
    }
    __syncthreads();
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int t = 32 * (cc >> 1) + 8 * (n >> 2) + 4 * (cc & 1) + (n & 3);
#pragma unroll
      for (int rt = 0; rt < 8; ++rt) {
        const int f = 8 * rt + 2 * g;
        const float2 x = kc[t * 64 + f], y = kc[t * 64 + f + 1];
        rot[cc][rt] = f16x4{(_Float16)x.x, (_Float16)x.y, (_Float16)y.x, (_Float16)y.y};
      }
    }
    __syncthreads();                                    // kc is overwritten by the u_k^T tiles below
    // u_k^T tiles: tile (rt, kb) lane (m, gg) element j = u_k[rank 32 kb + 8 gg + j][dim 16 rt + m]. Wave
    // w stages rank blocks kb = w, w + G2_NW, ...; its lane (gg, mh, rt) reads ranks 32 kb + 8 gg .. +7 at
    // dims 16 rt + 8 mh .. +7 (8 rows of 16 bytes; the wave reads 4 rows x 256 contiguous bytes per
    // step), transposes the 8 x 8 block in registers and writes 8 whole 16-byte tile slots. Rank blocks
    // past the group's r_k (a multiple of 32, so the test is uniform) are zero.
    {
      const int gg = lane & 3, mh = (lane >> 2) & 1, rt = lane >> 3;
      const __bf16* ukp = a.w_rot + (long long)kvh * a.rk * (2 * HD) + 16 * rt + 8 * mh;
      for (int kb = w; kb < KBP; kb += G2_NW) {
        bf16x8 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int r = 32 * kb + 8 * gg + j;
          v[j] = kb < KBe ? *reinterpret_cast<const bf16x8*>(ukp + (long long)r * (2 * HD)) : bf16x8{};
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          bf16x8 o;
#pragma unroll
          for (int j = 0; j < 8; ++j) o[j] = v[j][i];
          ukt[(rt * KBP + kb) * 64 + 16 * gg + 8 * mh + i] = o;
        }
      }
    }
    __syncthreads();
  }

  // Operand loads of a pair of blocks: register t[2 hb + c] of lane (n, g) holds rank indices
  // 32 kb + 8 g .. +7 of position 8 (n / 4) + 4 c + n % 4 of block 2 pp + hb (the B operand of the
  // rebuild). TILED: K-tile c * KB + kb of the block, one contiguous kilobyte. ROWS ([S, KW] row-major
  // stream): 16 bytes of that position's row, rows past the cache end clamped to its last row (their
  // scores are masked by the PV pass). Rank blocks past the group's r_k read kb 0 (the matching u_k^T
  // tiles are zero, and the cache columns past the group's rank are never touched); blocks past the
  // split's data read the split's first block. Every path issues the same loads.
  // The block and tile offsets are uniform (scalar registers), the lane's part the only vector one.
  auto load_kb = [&](int pp, int kb, bf16x8 (&t)[4]) {
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const int blk = 2 * pp + hb;
      const bool live = pp < npairs && blk < nblk;
      const int kbr = kb < KBe ? kb : 0;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        if constexpr (ROWS) {
          // a 32-bit byte offset from the uniform stream base (a stream holds at most 65536 x 512 values)
          const int p0 = __builtin_amdgcn_readfirstlane(s_lo + (live ? blk : 0) * BLK);
          const int p = min(p0 + lrow + 4 * c, a.S - 1);
          const uint32_t off = (uint32_t)(p * KW + 32 * kbr + 8 * g) * 2u;
          t[2 * hb + c] = *reinterpret_cast<const bf16x8*>(reinterpret_cast<const char*>(kbase) + off);
        } else {
          const long long off = __builtin_amdgcn_readfirstlane(
              (int)(((s_lo >> 5) + (live ? blk : 0)) * (32 * KB * 32) + (c * KB + kbr) * 512));
          t[2 * hb + c] = *reinterpret_cast<const bf16x8*>(kbase + off + lane * 8);
        }
      }
    }
  };

  // Query rotated back by the pair base, scaled by scale * log2 e, in fp16: qB[kq] is the B operand of the
  // QK MFMA over dims 32 kq + {4g .. 4g+3, 16+4g .. 16+4g+3} (the order of the packed K^T slices). The
  // angle of a frequency is the same for every head, so lane (n, g) composes only frequency
  // fi = 16 (n / 4) + 8 ((n / 2) % 2) + 2 g + n % 2 -- the 16 lanes of a DPP row (one g) hold the 16
  // frequencies that row's lanes use -- and takes the others' (cos, sin) by row broadcast.
  auto make_q = [&](int base, f16x8 (&qB)[4]) {
    const int J = base >> 6;
    const int fi = 16 * (n >> 2) + 8 * ((n >> 1) & 1) + 2 * g + (n & 1);
    const float2 l2 = tl[(J & 15) * 64 + fi];
    const float2 m2 = tm[((J >> 4) & 15) * 64 + fi];
    const float2 h2 = tt[(J >> 8) * 64 + fi];
    const float hc = h2.x * m2.x - h2.y * m2.y, hs = h2.y * m2.x + h2.x * m2.y;
    const float cf = hc * l2.x - hs * l2.y, sf = hs * l2.x + hc * l2.y;
    float4 qv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)                       // dims 32 (i / 2) + 16 (i % 2) + 4 g .. +3 of head n
      qv[i] = *reinterpret_cast<const float4*>(qs_lds + n * G_QS + 32 * (i >> 1) + 16 * (i & 1) + 4 * g);
    static_for<0, 16>([&](auto kc) {
      constexpr int k = decltype(kc)::value;          // frequency of row lane k: t = k / 4, half = (k / 2) % 2, p = k % 2
      constexpr int t = k >> 2, half = (k >> 1) & 1, p = k & 1;
      const float c = row_bcast<k>(cf), sn = row_bcast<k>(sf);
      const float4 q4 = qv[2 * t + half];
      const float x0 = p ? q4.z : q4.x, x1 = p ? q4.w : q4.y;
      qB[t][4 * half + 2 * p] = (_Float16)(x0 * c + x1 * sn);      // R_{-base}
      qB[t][4 * half + 2 * p + 1] = (_Float16)(x1 * c - x0 * sn);
    });
  };

  float* srow = scores + ((long long)(b * n_groups + grp) * NB + (s_lo >> 5)) * QH * BLK;
  bf16x8 ring[R][4];
#pragma unroll
  for (int kb = 0; kb < R; ++kb) load_kb(w, kb, ring[kb]);
  for (int pp = w; pp < npairs; pp += G2_NW) {
    f16x8 qB[4];
    make_q(s_lo + pp * 2 * BLK, qB);
    f32x4 acc[4][8];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc)
#pragma unroll
      for (int rt = 0; rt < 8; ++rt) acc[cc][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // u_k^T tiles double-buffered across rank blocks: the LDS reads of block kb + 1 are issued before
    // the MFMAs of block kb, so their latency hides behind them.
    bf16x8 A[2][8];
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) A[0][rt] = ukt[rt * KBP * 64 + lane];
#pragma unroll
    for (int kb = 0; kb < KBP; ++kb) {
      const int slot = kb % R;
      if (kb + 1 < KBP) {
#pragma unroll
        for (int rt = 0; rt < 8; ++rt) A[(kb + 1) & 1][rt] = ukt[(rt * KBP + kb + 1) * 64 + lane];
      }
#pragma unroll
      for (int rt = 0; rt < 8; ++rt)
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) acc[cc][rt] = mfma16(A[kb & 1][rt], ring[slot][cc], acc[cc][rt]);
      if (kb + R < KBP) load_kb(pp, kb + R, ring[slot]);
      else load_kb(pp + G2_NW, kb + R - KBP, ring[slot]);
      __builtin_amdgcn_sched_barrier(0);                 // keep the reads of one rank block ahead, not more
    }
    // Rotate in packed fp16 ((x0, x1) * (c, c) + (x1, x0) * (-s, s)), then contract each 32-dim slice
    // with the query on the fp16 MFMA: scores of 16 positions x 16 heads per (block, tile c).
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kq = 0; kq < 4; ++kq) {
        f16x2 r[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int rt = 2 * kq + h;
          // The empty asm keeps the table in its compact form: built here, (c, c) and (-s, s) fold into
          // the packed ops' operand selects and negations; hoisted, they would double its registers.
          f16x4 t = rot[cc][rt];
          asm volatile("" : "+v"(t));
          const f16x2 c0 = {t[0], t[0]}, s0 = {-t[1], t[1]}, c1 = {t[2], t[2]}, s1 = {-t[3], t[3]};
          const f16x2 x01 = to_f16x2(acc[cc][rt][0], acc[cc][rt][1]);
          const f16x2 x23 = to_f16x2(acc[cc][rt][2], acc[cc][rt][3]);
          r[h][0] = x01 * c0 + x01.yx * s0;
          r[h][1] = x23 * c1 + x23.yx * s1;
        }
        const f16x8 kA = {r[0][0][0], r[0][0][1], r[0][1][0], r[0][1][1], r[1][0][0], r[1][0][1], r[1][1][0], r[1][1][1]};
        sc = mfma16(kA, qB[kq], sc);
      }
      const int hb = cc >> 1, c = cc & 1;
      const int blk = 2 * pp + hb;
      // lane (head n, g) holds positions 8g + 4c .. +3 of block blk
      if (blk < nblk && n < a.rep)
        *reinterpret_cast<float4*>(srow + ((long long)blk * QH + hig * a.rep + n) * BLK + 8 * g + 4 * c) =
            make_float4(sc[0], sc[1], sc[2], sc[3]);
    }
  }
}

template <int KBP, typename TabT, bool ROWS>
int launch_scores_full(const DecodeArgs& a, float* scores, int n_wg, hipStream_t stream) {
  auto kern = palu_glrd_scores_full_kernel<KBP, TabT, ROWS>;
  const int lds = G2Smem<KBP>::BYTES;
  static int attr_set = 0;
  if (attr_set < lds) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return fail(PALU_EHIP, "hipFuncSetAttribute: %s", hipGetErrorString(e));
    attr_set = lds;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)n_wg), dim3(G2_NW * 64), lds, stream, a, scores);
  return PALU_OK;
}

}  // namespace

namespace palu {

// Launches the scores kernel for a K rank of at most 256 (rank blocks rounded up to even, 2 .. 8);
// defined in palu_glrd_narrow.hip.
int glrd_scores_narrow(const DecodeArgs& a, float* scores, int n_wg, hipStream_t s, bool rows, bool tab_f32);

}  // namespace palu
