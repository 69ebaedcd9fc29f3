// Decode-step projections: y[m][c] = sum_k x[m][k] w[c][k] for the rows of one decode step (m <= 64),
// bf16 in, fp32 accumulate. Every weight byte is used once per step by all m rows, so each call is one
// stream of the weight matrix from HBM; the activations (at most 64 x k bf16, L2-resident) are re-read
// from L2 by every workgroup. No counterpart in the reference's op interface: these are the
// ttnn.linear calls of the reference model's decode step (palu_tt/attention.py:585-733, model.py),
// which the decoder issues for its QKV, output, gate/up, down and LM-head projections.
//
// Weights are stored tiled (palu_tt.decoder_ops.tile_weight): row tile rt (16 output columns) and k
// tile kt (32 inputs) form one 1 KB tile, the A operand of v_mfma_f32_16x16x32_bf16 for one wave, lane
// l = 16 g + n holding w[16 rt + n][32 kt + 8 g .. +7]. Row tiles form groups of RTW (the last group may
// be shorter) and a group's tiles are stored k tile by k tile ([kt][rt in group]), so the workgroup that
// owns a group (or one k slice of it) reads one sequential stream; every weight load of a wave is one
// aligned kilobyte. The activations come row-major (lane (g, n) of tile (kt, mt) reads 16 bytes of row
// 16 mt + n: sixteen half cache lines per tile) or tiled the same way as the weights with the 64 rows as
// four row tiles ([kt][mt], palu_tt.decoder_ops.tile_rows; one contiguous kilobyte per tile), which
// the decoder's RMSNorm and SwiGLU kernels write directly.
//
// Outputs (the epilogue, EPI): bf16 y [m][n] (split partials summed by a second launch); the fp32 split
// partials [KS][m][n] themselves, for a consumer that sums them (palu_rmsnorm's residual input,
// palu_qkv_post); for a gate / up weight interleaved eight rows at a time (tile_weight of
// palu_tt.decoder_ops.interleave_gate_up), silu(gate) * up in the tiled activation layout, optionally
// of the RMS-normalised x (the row scale rsqrt(mean(x^2) + eps) applied to the products, the norm's
// weight folded into the gate / up weight; the loop sums x^2 from the activation tiles it already
// loads); the residual update h += y, also written tiled for the next projection; or the decode step's
// QKV epilogue (q RoPE, K / V latent appends), in place of palu_qkv_post's second launch. The last three
// need KS = 1: the epilogue sees whole dot products.
//
// A workgroup owns one group and one of KS slices of the k tiles. Its 4 waves (one per SIMD, so each may
// use the whole 512-entry register file) take the slice's k tiles in turn (wave w: kt0 + w, kt0 + w + 4,
// ...). Per k tile a wave loads RTW weight tiles (nontemporal: read once per step) and the four 16-row
// activation tiles (cached), and issues RTW x 4 MFMAs into RTW x 4 accumulators; the loads of the next
// NB - 1 k tiles are in flight meanwhile. The waves' partial sums meet in LDS, and each wave adds up and
// stores a quarter of the output tiles (bf16 y, fp32 split partials, or the SwiGLU activations).
//
// Measured on MI355X (64 rows, weights rotated past the MALL, HIP-graph launches): the tiled activations
// take the gate/up projection (28672 x 4096) from 51.9 to 43.4 us, against 52.5 us for hipBLASLt; a
// copy of this loop with the MFMAs and activation loads removed streams the weights at 5.6-5.9 TB/s,
// and deeper buffering (6 or 8 steps) or 8 waves per workgroup did not raise it.
#include "palu_kernel.h"

namespace {

constexpr int LIN_MT = 4;                       // 16-row activation tiles: m <= 64
constexpr int LIN_MAX_RTW = 8;

// Epilogues.
constexpr int EPI_OUT = 0;           // bf16 y, or the fp32 split partials
constexpr int EPI_SWIGLU = 1;        // silu(gate) * up, tiled
constexpr int EPI_SWIGLU_NORM = 2;   // the same over RMS-normalised x
constexpr int EPI_RESID = 3;         // h += y (row-major), and h tiled
constexpr int EPI_QKV = 4;           // q RoPE and latent appends (QkvEpi)

struct LinEpi {
  float eps, inv_k;                  // EPI_SWIGLU_NORM
  __bf16* h;                         // EPI_RESID: [m][n] bf16, rows ldh apart
  long long ldh;
  __bf16* h_tiled;                   //   and the 64-row tiled copy (or null)
  QkvEpi q;                          // EPI_QKV
};

template <int RTW, int NW, int EPI>
struct LinSmem {
  static constexpr int SLOT = RTW * LIN_MT * 64;          // f32x4 per wave partial
  static constexpr int RED = NW * SLOT * 16;              // every wave's partial
  static constexpr int BYTES = RED + (EPI == EPI_SWIGLU_NORM ? NW * 64 * 4 : 0);   // + per-wave row sums of x^2
};

// Where the QKV epilogue sends columns col .. col + 3: kind 0 (q head gi), 1 / 2 (group gi's K / V
// slice) at column c of the head or slice, or -1 (a column no part reads).
__device__ __forceinline__ int qkv_part_of(const QkvEpi& e, int col, int& gi, int& c) {
  gi = 0;
  c = 0;
  if (col < e.nh * HD) {
    gi = col / HD;
    c = col - gi * HD;
    return 0;
  }
  if (col >= e.k_off && col < e.k_off + (e.G - 1) * e.k_gs + e.k_w) {
    const int d = col - e.k_off;
    gi = e.G > 1 ? d / e.k_gs : 0;
    c = d - gi * e.k_gs;
    return c < e.k_w ? 1 : -1;
  }
  if (col >= e.v_off && col < e.v_off + (e.G - 1) * e.v_gs + e.v_w) {
    const int d = col - e.v_off;
    gi = e.G > 1 ? d / e.v_gs : 0;
    c = d - gi * e.v_gs;
    return c < e.v_w ? 2 : -1;
  }
  return -1;
}

// NB register buffers per wave, so each step's loads are issued NB - 1 steps before its MFMAs. Weight
// and activation tiles of one step share a buffer: loads return in issue order, so an activation tile
// loaded later than the weights would make every wait a wait for those weights too. NW waves per
// workgroup (the launches use 4: one per SIMD, the whole register file each; 8, two per SIMD, was slower
// end to end for the one- and two-tile projections).
template <int RTW, int NB, int NW, bool XT, int EPI>
__global__ __launch_bounds__(NW * 64) void palu_linear_kernel(const __bf16* __restrict__ x, long long ldx, int m,
                                                              const __bf16* __restrict__ wt, int n16, int kt_total,
                                                              int ks_count, int kt_per_split,
                                                              __bf16* __restrict__ y, long long ldy,
                                                              float* __restrict__ part, const LinEpi ep) {
  using SM = LinSmem<RTW, NW, EPI>;
  constexpr bool SWIGLU = EPI == EPI_SWIGLU || EPI == EPI_SWIGLU_NORM;
  constexpr int NT = (RTW * LIN_MT + NW - 1) / NW;       // output tiles each wave stores (at most)
  extern __shared__ __attribute__((aligned(16))) char smem[];
  f32x4* red = reinterpret_cast<f32x4*>(smem);

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int mm = lane & 15, g = lane >> 4;
  const int ks = blockIdx.x % ks_count;
  const int rt0 = (blockIdx.x / ks_count) * RTW;
  const int rt_cnt = min(RTW, n16 - rt0);                 // uniform: the last group may be short
  const int kt_lo = ks * kt_per_split;
  const int kt_hi = min(kt_total, kt_lo + kt_per_split);

  // The epilogue's own global reads (the residual h, the rows' positions) are issued here, ahead of the
  // weight stream, so the epilogue does not start with a round trip to memory. Wave w stores output
  // tiles t = w, w + NW, ... (row tile t / 4, activation tile t % 4); lane (g, mm) of tile t holds
  // columns 16 (rt0 + t / 4) + 4 g .. + 3 of row 16 (t % 4) + mm.
  bf16x4 hpre[NT];
  int ppre[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    const int t = w + i * NW;
    const int r = t / LIN_MT, row = 16 * (t % LIN_MT) + mm;
    const bool ok = t < RTW * LIN_MT && r < rt_cnt && row < m;
    if constexpr (EPI == EPI_RESID) {
      const int col = 16 * (rt0 + (ok ? r : 0)) + 4 * g;
      hpre[i] = *reinterpret_cast<const bf16x4*>(ep.h + (ok ? row : 0) * ep.ldh + col);
    }
    if constexpr (EPI == EPI_QKV) ppre[i] = ep.q.pos[ok ? row : 0];
  }

  // Activation rows past m are replaced by zeros (row-major: they read row 0); their outputs are not
  // stored.
  const __bf16* xp[LIN_MT];
  bool xv[LIN_MT];
#pragma unroll
  for (int mt = 0; mt < LIN_MT; ++mt) {
    const int r = 16 * mt + mm;
    xv[mt] = r < m;
    xp[mt] = XT ? x + ((long long)mt * 64 + lane) * 8 : x + (long long)(xv[mt] ? r : 0) * ldx + 8 * g;
  }
  const bf16x8* wp = reinterpret_cast<const bf16x8*>(wt) + (long long)rt0 * kt_total * 64 + lane;

  f32x4 acc[RTW][LIN_MT];
#pragma unroll
  for (int r = 0; r < RTW; ++r)
#pragma unroll
    for (int mt = 0; mt < LIN_MT; ++mt) acc[r][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float ss[LIN_MT] = {0.f, 0.f, 0.f, 0.f};              // EPI_SWIGLU_NORM: this lane's share of sum x^2 per row

  // Every load is issued on every path (row tiles past rt_cnt read the last row tile, k tiles past the
  // slice read the matrix's last k tile; their products are never stored), so each wait in the loop is
  // for exactly the loads of the buffer about to be used.
  bf16x8 wa[NB][RTW], xb[NB][LIN_MT];
  // Every workgroup reads the same activation tiles. Walked in the same order, all workgroups would
  // request the same few kilobytes at once; instead each group starts its slice at its own offset and
  // wraps around (32-layer decode step 5.21 -> 5.16 ms in a same-box A/B). i -> (i + krot) mod klen is
  // a permutation of the slice, so the waves together still cover each k tile once; the sums are the
  // same up to the order of the fp32 additions.
  const int klen = kt_hi - kt_lo;
  const int kper = klen / NW > 0 ? klen / NW : 1;
  const int krot = ((blockIdx.x / ks_count) * 37 % kper) * NW % (klen > 0 ? klen : 1);
  auto load = [&](int buf, int kt) {
    int i = kt - kt_lo;                                   // steps past the slice read its last tile
    i = i < klen ? (i + krot >= klen ? i + krot - klen : i + krot) : klen - 1;
    kt = klen > 0 ? min(kt_lo + i, kt_total - 1) : kt_total - 1;   // an empty slice reads the last tile
#pragma unroll
    for (int r = 0; r < RTW; ++r)
      wa[buf][r] = __builtin_nontemporal_load(wp + ((long long)kt * rt_cnt + min(r, rt_cnt - 1)) * 64);
#pragma unroll
    for (int mt = 0; mt < LIN_MT; ++mt)
      xb[buf][mt] = *reinterpret_cast<const bf16x8*>(xp[mt] + (XT ? (long long)kt * (LIN_MT * 512) : 32LL * kt));
  };
  auto compute = [&](int buf, bool live) {
    bf16x8 bz[LIN_MT];
#pragma unroll
    for (int mt = 0; mt < LIN_MT; ++mt) bz[mt] = (xv[mt] && live) ? xb[buf][mt] : bf16x8{};
#pragma unroll
    for (int r = 0; r < RTW; ++r)
#pragma unroll
      for (int mt = 0; mt < LIN_MT; ++mt) acc[r][mt] = mfma16(wa[buf][r], bz[mt], acc[r][mt]);
    if constexpr (EPI == EPI_SWIGLU_NORM) {
      // x^2 summed in pairs (v_dot2: the bf16 products are exact in fp32)
#pragma unroll
      for (int mt = 0; mt < LIN_MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bf16x2 p2{bz[mt][2 * j], bz[mt][2 * j + 1]};
          ss[mt] = __builtin_amdgcn_fdot2_f32_bf16(p2, p2, ss[mt], false);
        }
    }
  };

  // The loop is unrolled by NB so that buffer indices are compile-time, and has no branch: steps past the
  // wave's count (the rest of the last round) load clamped tiles and multiply them by zero activations.
  // The scheduling barriers keep each step's loads ahead of the earlier step's MFMAs (left alone, the
  // compiler sinks every load to its first use and the wave has one tile in flight).
  // The prologue's loads keep their order (a scheduling barrier after each buffer): the loop-top wait
  // is computed from the load order on both paths into the loop, and a prologue reordered by the
  // scheduler made the compiler wait there for all but the newest loads, a drain every NB steps
  // (32-layer decode step 5.27 -> 5.23 ms in a same-box A/B).
  const int kt0 = kt_lo + w;
  const int nsteps = kt0 < kt_hi ? (kt_hi - kt0 + NW - 1) / NW : 0;   // uniform per wave
#pragma unroll
  for (int j = 0; j < NB - 1; ++j) {
    load(j, kt0 + j * NW);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int s = 0; s < nsteps; s += NB) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      load((j + NB - 1) % NB, kt0 + (s + j + NB - 1) * NW);
      __builtin_amdgcn_sched_barrier(0);
      compute(j, s + j < nsteps);
    }
  }

  // The waves' partials meet in LDS (slot layout [wave][r][mt][lane] of f32x4); each wave then sums
  // the NW slots of every NW-th (r, mt) tile and stores that tile, so the epilogue's arithmetic and
  // stores are spread over the SIMDs. Every LDS read of the sums is issued before the first is used and
  // the tiles are stored under a predicate rather than a branch per tile: the epilogue sits between the
  // last weight load and the end of the launch, and one round trip to LDS per tile (its reads, then the
  // next tile's) made it 1.2 us longer for the gate / up shape.
#pragma unroll
  for (int r = 0; r < RTW; ++r)
#pragma unroll
    for (int mt = 0; mt < LIN_MT; ++mt) red[w * SM::SLOT + (r * LIN_MT + mt) * 64 + lane] = acc[r][mt];
  float* rss = reinterpret_cast<float*>(smem + SM::RED);   // [wave][row] sums of x^2
  if constexpr (EPI == EPI_SWIGLU_NORM) {
    // lanes (g, mm), g = 0..3, hold columns 8 g .. 8 g + 7 of every k tile of row 16 mt + mm
    float s16[LIN_MT];
#pragma unroll
    for (int mt = 0; mt < LIN_MT; ++mt) s16[mt] = ss[mt] + __shfl_xor(ss[mt], 16, 64);
#pragma unroll
    for (int mt = 0; mt < LIN_MT; ++mt) ss[mt] = s16[mt] + __shfl_xor(s16[mt], 32, 64);
    if (g == 0) {
#pragma unroll
      for (int mt = 0; mt < LIN_MT; ++mt) rss[w * 64 + 16 * mt + mm] = ss[mt];
    }
  }
  __syncthreads();

  // Wave w's tiles t = w + i NW, i < NT (clamped to the last tile for the loads; tiles past it are not
  // stored). Lane (g, mm) of tile (r, mt) holds y^T[16 (rt0 + r) + 4 g + i][16 mt + mm], i < 4: four
  // consecutive output columns of activation row 16 mt + mm.
  f32x4 v[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    const int t = min(w + i * NW, RTW * LIN_MT - 1);
    v[i] = red[t * 64 + lane];
#pragma unroll
    for (int q = 1; q < NW; ++q) v[i] += red[q * SM::SLOT + t * 64 + lane];
  }
  if constexpr (EPI == EPI_SWIGLU_NORM) {
    // the row scale rsqrt(mean x^2 + eps): with NW a multiple of LIN_MT (asserted below) every tile of
    // wave w lies in activation tile w % LIN_MT, one row per lane
    const int row = 16 * (w % LIN_MT) + mm;
    float tot = 0.f;
#pragma unroll
    for (int q = 0; q < NW; ++q) tot += rss[q * 64 + row];
    const float sc = rsqrtf(tot * ep.inv_k + ep.eps);
#pragma unroll
    for (int i = 0; i < NT; ++i) v[i] *= sc;
  }
  if constexpr (SWIGLU) {
    static_assert(NW % LIN_MT == 0, "the SwiGLU epilogue pairs tiles of one activation tile");
    // Gate / up pairs: rows 0-7 of row tile rt are gate columns 8 rt .. 8 rt + 7 and rows 8-15 the up
    // columns of the same outputs (tile_weight of the interleaved weight), so lanes g < 2 of a tile hold
    // gate values and lanes g + 2, 32 lanes on, the matching up values. Tiles i and i + 1 of a wave
    // share their activation rows; one v_permlane32_swap of the upper half of tile i with the lower half
    // of tile i + 1 puts the gates of both in one register and the ups in the other, so that every lane
    // computes and stores one output of one of the two tiles (lanes 32-63: tile i + 1, output columns
    // 8 rt + 4 (g - 2) .. + 3). out = silu(gate) * up, stored in the tiled activation layout (64 rows x
    // n / 2) the next projection reads.
    const int row = 16 * (w % LIN_MT) + mm;
#pragma unroll
    for (int i = 0; i < NT; i += 2) {
      const int j = i + 1 < NT ? i + 1 : i;
      f32x4 gv, uv;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i][k]), __float_as_uint(v[j][k]), false, false);
        gv[k] = __uint_as_float(sw[0]);
        uv[k] = __uint_as_float(sw[1]);
      }
      bf16x4 o;
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = (__bf16)((gv[k] / (1.f + __expf(-gv[k]))) * uv[k]);
      const int t = w + (g < 2 ? i : j) * NW, r = t / LIN_MT;
      if (t < RTW * LIN_MT && r < rt_cnt && row < m && (g < 2 || j != i))
        *reinterpret_cast<bf16x4*>(y + tiled_row_offset(row, 8 * (rt0 + r) + 4 * (g & 1))) = o;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      const int t = w + i * NW;
      const int r = t / LIN_MT, row = 16 * (t % LIN_MT) + mm;
      const bool ok = t < RTW * LIN_MT && r < rt_cnt && row < m;
      if constexpr (EPI == EPI_RESID) {
        // h + y rounded to bf16 once (the residual stream), in place and in the tiled layout
        if (ok) {
          const int col = 16 * (rt0 + r) + 4 * g;
          bf16x4 o;
#pragma unroll
          for (int k = 0; k < 4; ++k) o[k] = (__bf16)((float)hpre[i][k] + v[i][k]);
          *reinterpret_cast<bf16x4*>(ep.h + row * ep.ldh + col) = o;
          if (ep.h_tiled) *reinterpret_cast<bf16x4*>(ep.h_tiled + tiled_row_offset(row, col)) = o;
        }
      } else if constexpr (EPI == EPI_QKV) {
        // Columns col .. col + 3 of QKV row `row` lie in one q head or one group's K or V slice (the
        // entry point checks that the three ranges do not overlap and start on multiples of 8).
        int gi, c;
        const int kind = ok ? qkv_part_of(ep.q, 16 * (rt0 + r) + 4 * g, gi, c) : -1;
        if (kind >= 0) {
          float vv[4] = {v[i][0], v[i][1], v[i][2], v[i][3]};
          qkv_store<4>(ep.q, row, ppre[i], kind, gi, c, vv);
        }
      } else {
        if (ok) {
          const long long col = 16LL * (rt0 + r) + 4 * g;
          if (part) {
            *reinterpret_cast<f32x4*>(part + ((long long)ks * m + row) * (16LL * n16) + col) = v[i];
          } else {
            bf16x4 o;
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = (__bf16)v[i][k];
            *reinterpret_cast<bf16x4*>(y + row * ldy + col) = o;
          }
        }
      }
    }
  }
}

// Greedy pick fused into the LM head: for y = x w^T (one k slice, the sums and their order those of
// palu_linear_kernel, rounded to bf16 as its plain output would be), key[r][wg] = the largest
// (value, -column) of row r over the columns of every group workgroup wg ran, packed so that one
// unsigned 64-bit max picks the largest value and, among equal ones, the first column: bits 63-32 the
// bf16 value made order-preserving (NaN above +inf, -0 taken as +0), bits 31-0 ~column. The max is
// associative, so a workgroup keeps one running key per row over its groups and stores it once, at the
// end (stores inside the group loop would hold the next group's loads behind them: the loop's waits
// count stores too). palu_argmax_keys_kernel then reduces a row's workgroup keys. The logits are never written: at the LM head's shape (64 x 128256) the 16 MB of bf16
// stores cost the projection 30 us of its 191 (a probe with the same loop and one 8-byte store per
// lane and group: 175-183 us), and the argmax launch that read them back 11.5 us.
// A fixed grid of at most PERSIST_WGS workgroups takes groups blockIdx.x, blockIdx.x + gridDim.x, ...;
// the next group's first NB - 1 k steps are issued before the current group's LDS reduce and key
// stores, so the weight stream runs on through them.
constexpr int PERSIST_WGS = 256;

__device__ __forceinline__ unsigned long long argmax_key(float v, int col) {
  unsigned u = __builtin_bit_cast(unsigned short, (__bf16)v);
  if ((u & 0x7fffu) > 0x7f80u) u = 0xffffu;                   // NaN: above every number
  else if ((u & 0x7fffu) == 0) u = 0x8000u;                   // -0 and +0 compare equal
  else u = (u & 0x8000u) ? (~u & 0xffffu) : (u | 0x8000u);
  return ((unsigned long long)u << 32) | (0xffffffffu - (unsigned)col);
}

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long v, int mask) {
  const unsigned lo = __shfl_xor((unsigned)v, mask, 64), hi = __shfl_xor((unsigned)(v >> 32), mask, 64);
  return ((unsigned long long)hi << 32) | lo;
}

template <int RTW, int NB, int NW, bool XT>
__global__ __launch_bounds__(NW * 64) void palu_linear_argmax_kernel(const __bf16* __restrict__ x, long long ldx,
                                                                     int m, const __bf16* __restrict__ wt, int n16,
                                                                     int kt_total,
                                                                     unsigned long long* __restrict__ keys) {
  using SM = LinSmem<RTW, NW, EPI_OUT>;
  static_assert(NW == LIN_MT, "wave w reduces activation rows 16 w .. 16 w + 15");
  constexpr int NT = (RTW * LIN_MT + NW - 1) / NW;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  f32x4* red = reinterpret_cast<f32x4*>(smem);
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int mm = lane & 15, g = lane >> 4;
  const int groups = (n16 + RTW - 1) / RTW;

  const __bf16* xp[LIN_MT];
  bool xv[LIN_MT];
#pragma unroll
  for (int mt = 0; mt < LIN_MT; ++mt) {
    const int r = 16 * mt + mm;
    xv[mt] = r < m;
    xp[mt] = XT ? x + ((long long)mt * 64 + lane) * 8 : x + (long long)(xv[mt] ? r : 0) * ldx + 8 * g;
  }
  // The group a workgroup streams: its row tiles and its k offset (palu_linear_kernel's, one slice).
  const int klen = kt_total;
  const int kper = klen / NW > 0 ? klen / NW : 1;
  int grp = blockIdx.x;
  int rt0 = 0, rt_cnt = 0, krot = 0;
  const bf16x8* wp = nullptr;
  auto setup = [&](int gi) {
    gi = gi < groups ? gi : groups - 1;                  // past the last group: reload it (never reduced)
    rt0 = gi * RTW;
    rt_cnt = min(RTW, n16 - rt0);
    krot = (gi * 37 % kper) * NW % klen;
    wp = reinterpret_cast<const bf16x8*>(wt) + (long long)rt0 * kt_total * 64 + lane;
  };
  setup(grp);
  unsigned long long best = 0;                              // below every key (no value maps to 0)

  bf16x8 wa[NB][RTW], xb[NB][LIN_MT];
  auto load = [&](int buf, int kt) {
    int i = kt < klen ? (kt + krot >= klen ? kt + krot - klen : kt + krot) : klen - 1;
#pragma unroll
    for (int r = 0; r < RTW; ++r) wa[buf][r] = __builtin_nontemporal_load(wp + ((long long)i * rt_cnt + min(r, rt_cnt - 1)) * 64);
#pragma unroll
    for (int mt = 0; mt < LIN_MT; ++mt)
      xb[buf][mt] = *reinterpret_cast<const bf16x8*>(xp[mt] + (XT ? (long long)i * (LIN_MT * 512) : 32LL * i));
  };
  const int kt0 = w;
  const int nsteps = kt0 < klen ? (klen - kt0 + NW - 1) / NW : 0;
#pragma unroll
  for (int j = 0; j < NB - 1; ++j) {
    load(j, kt0 + j * NW);
    __builtin_amdgcn_sched_barrier(0);
  }
  while (true) {
    f32x4 acc[RTW][LIN_MT];
#pragma unroll
    for (int r = 0; r < RTW; ++r)
#pragma unroll
      for (int mt = 0; mt < LIN_MT; ++mt) acc[r][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < nsteps; s += NB) {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        load((j + NB - 1) % NB, kt0 + (s + j + NB - 1) * NW);
        __builtin_amdgcn_sched_barrier(0);
        bf16x8 bz[LIN_MT];
#pragma unroll
        for (int mt = 0; mt < LIN_MT; ++mt) bz[mt] = (xv[mt] && s + j < nsteps) ? xb[j][mt] : bf16x8{};
#pragma unroll
        for (int r = 0; r < RTW; ++r)
#pragma unroll
          for (int mt = 0; mt < LIN_MT; ++mt) acc[r][mt] = mfma16(wa[j][r], bz[mt], acc[r][mt]);
      }
    }
    // This group's sums to LDS (after every wave has read the previous group's), then the next group's
    // first k steps go out before the reads and the key stores of this one.
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RTW; ++r)
#pragma unroll
      for (int mt = 0; mt < LIN_MT; ++mt) red[w * SM::SLOT + (r * LIN_MT + mt) * 64 + lane] = acc[r][mt];
    const int cur_rt0 = rt0, cur_rt_cnt = rt_cnt;
    const int next = grp + (int)gridDim.x;                 // uniform
    setup(next);
#pragma unroll
    for (int j = 0; j < NB - 1; ++j) {
      load(j, kt0 + j * NW);
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
    // Wave w's tiles t = w + i NW are row tiles r = i of activation rows 16 w + mm; lane (g, mm) holds
    // columns 16 (rt0 + i) + 4 g .. + 3 of row 16 w + mm.
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      const int t = min(w + i * NW, RTW * LIN_MT - 1);
      f32x4 v = red[t * 64 + lane];
#pragma unroll
      for (int q = 1; q < NW; ++q) v += red[q * SM::SLOT + t * 64 + lane];
      if (w + i * NW < RTW * LIN_MT && i < cur_rt_cnt) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const unsigned long long key = argmax_key(v[k], 16 * (cur_rt0 + i) + 4 * g + k);
          best = key > best ? key : best;
        }
      }
    }
    if (next >= groups) break;
    grp = next;
  }
  unsigned long long o = shfl_xor_u64(best, 16);
  best = o > best ? o : best;
  o = shfl_xor_u64(best, 32);
  best = o > best ? o : best;
  const int row = 16 * w + mm;
  if (g == 0 && row < m) keys[(long long)row * gridDim.x + blockIdx.x] = best;
}

// ids[r] = the column of the largest of row r's n_keys keys (one workgroup per row).
__global__ __launch_bounds__(256) void palu_argmax_keys_kernel(const unsigned long long* __restrict__ keys, int n_keys,
                                                               long long* __restrict__ ids) {
  __shared__ unsigned long long part[4];
  const int row = blockIdx.x;
  unsigned long long best = 0;
  for (int gi = threadIdx.x; gi < n_keys; gi += 256) {
    const unsigned long long k = keys[(long long)row * n_keys + gi];
    best = k > best ? k : best;
  }
#pragma unroll
  for (int mask = 32; mask >= 1; mask >>= 1) {
    const unsigned long long o = shfl_xor_u64(best, mask);
    best = o > best ? o : best;
  }
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int q = 1; q < 4; ++q) best = part[q] > best ? part[q] : best;
    ids[row] = (long long)(0xffffffffu - (unsigned)(best & 0xffffffffu));
  }
}

template <int RTW, bool XT>
hipError_t launch_argmax_cfg(const __bf16* x, long long ldx, int m, const __bf16* wt, int n16, int kt_total,
                             unsigned long long* keys, long long* ids, hipStream_t s) {
  constexpr int NB = 4;
  constexpr int NW = 4;
  auto kern = palu_linear_argmax_kernel<RTW, NB, NW, XT>;
  constexpr int lds = LinSmem<RTW, NW, EPI_OUT>::BYTES;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int groups = (n16 + RTW - 1) / RTW;
  const int n_wg = std::min(groups, PERSIST_WGS);          // one key per row and workgroup
  hipLaunchKernelGGL(kern, dim3(n_wg), dim3(NW * 64), lds, s, x, ldx, m, wt, n16, kt_total, keys);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  hipLaunchKernelGGL(palu_argmax_keys_kernel, dim3(m), dim3(256), 0, s, keys, n_wg, ids);
  return hipGetLastError();
}

template <bool XT>
hipError_t launch_argmax(int rtw, const __bf16* x, long long ldx, int m, const __bf16* wt, int n16, int kt_total,
                         unsigned long long* keys, long long* ids, hipStream_t s) {
  switch (rtw) {
    case 1: return launch_argmax_cfg<1, XT>(x, ldx, m, wt, n16, kt_total, keys, ids, s);
    case 2: return launch_argmax_cfg<2, XT>(x, ldx, m, wt, n16, kt_total, keys, ids, s);
    case 3: return launch_argmax_cfg<3, XT>(x, ldx, m, wt, n16, kt_total, keys, ids, s);
    case 4: return launch_argmax_cfg<4, XT>(x, ldx, m, wt, n16, kt_total, keys, ids, s);
    case 5: return launch_argmax_cfg<5, XT>(x, ldx, m, wt, n16, kt_total, keys, ids, s);
    case 6: return launch_argmax_cfg<6, XT>(x, ldx, m, wt, n16, kt_total, keys, ids, s);
    case 7: return launch_argmax_cfg<7, XT>(x, ldx, m, wt, n16, kt_total, keys, ids, s);
    default: return launch_argmax_cfg<8, XT>(x, ldx, m, wt, n16, kt_total, keys, ids, s);
  }
}

// y[r][c] = bf16(sum over ks of part[ks][r][c]); 4 columns per thread.
__global__ __launch_bounds__(256) void palu_linear_reduce_kernel(const float* __restrict__ part, int ks_count, int m,
                                                                 int n, __bf16* __restrict__ y, long long ldy) {
  const long long quads = (long long)m * (n / 4);
  for (long long e = blockIdx.x * 256LL + threadIdx.x; e < quads; e += (long long)gridDim.x * 256) {
    const int r = (int)(e / (n / 4)), c = (int)(e % (n / 4)) * 4;
    f32x4 s = *reinterpret_cast<const f32x4*>(part + (long long)r * n + c);
    for (int k = 1; k < ks_count; ++k) s += *reinterpret_cast<const f32x4*>(part + ((long long)k * m + r) * n + c);
    bf16x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (__bf16)s[i];
    *reinterpret_cast<bf16x4*>(y + r * ldy + c) = o;
  }
}

// Register buffers per wave: NB = 4 for every width. Workgroups of one or two row tiles load more
// activation than weight bytes per k tile (4 KB against 1-2 KB), and deeper rings only queue more of
// those L2 reads ahead of the weights: in graph-captured probes the QKV shape (two row tiles) took 16.4 us
// at NB 4 against 17.0 at 8 and 18.2 at 12, the output projection's (one row tile) 7.9 against 8.2 us at 8,
// and the 32-layer decode step 5.02 against 5.06 ms (same-box A/B, three runs each).

template <int RTW, bool XT, int EPI>
hipError_t launch_cfg(const __bf16* x, long long ldx, int m, const __bf16* wt, int n16, int kt_total, int ks,
                      int ktps, __bf16* y, long long ldy, float* part, const LinEpi& ep, hipStream_t s) {
  constexpr int NB = 4;
  constexpr int NW = 4;                                   // one wave per SIMD (8 measured slower end to end)
  auto kern = palu_linear_kernel<RTW, NB, NW, XT, EPI>;
  constexpr int lds = LinSmem<RTW, NW, EPI>::BYTES;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int groups = (n16 + RTW - 1) / RTW;
  hipLaunchKernelGGL(kern, dim3(groups * ks), dim3(NW * 64), lds, s, x, ldx, m, wt, n16, kt_total, ks, ktps, y,
                     ldy, part, ep);
  return hipGetLastError();
}

template <bool XT, int EPI>
hipError_t launch_rtw(int rtw, const __bf16* x, long long ldx, int m, const __bf16* wt, int n16, int kt_total, int ks,
                      int ktps, __bf16* y, long long ldy, float* part, const LinEpi& ep, hipStream_t s) {
  switch (rtw) {
    case 1: return launch_cfg<1, XT, EPI>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, ep, s);
    case 2: return launch_cfg<2, XT, EPI>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, ep, s);
    case 3: return launch_cfg<3, XT, EPI>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, ep, s);
    case 4: return launch_cfg<4, XT, EPI>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, ep, s);
    case 5: return launch_cfg<5, XT, EPI>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, ep, s);
    case 6: return launch_cfg<6, XT, EPI>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, ep, s);
    case 7: return launch_cfg<7, XT, EPI>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, ep, s);
    default: return launch_cfg<8, XT, EPI>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, ep, s);
  }
}

template <int EPI>
hipError_t launch_epi(int x_tiled, int rtw, const __bf16* x, long long ldx, int m, const __bf16* wt, int n16,
                      int kt_total, int ks, int ktps, __bf16* y, long long ldy, float* part, const LinEpi& ep,
                      hipStream_t s) {
  return x_tiled ? launch_rtw<true, EPI>(rtw, x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, ep, s)
                 : launch_rtw<false, EPI>(rtw, x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, ep, s);
}

// Row tiles per workgroup and k slices: the pair whose busiest CU streams the fewest bytes, counting the
// activation re-reads (4 KB per k tile and workgroup, from L2, weighted at a quarter of a weight byte)
// and the split partials (written and read once in fp32, weighted at three weight bytes each: measured,
// the k-split passes cost more than their bytes).
void plan(int m, int n16, int kt_total, int max_ks, int* rtw_out, int* ks_out) {
  constexpr int CUS = 256;
  double best = 1e300;
  int br = 1, bk = 1;
  for (int rtw = 1; rtw <= LIN_MAX_RTW; ++rtw) {
    for (int ks = 1; ks <= 16 && ks <= max_ks; ks *= 2) {
      const int ktps = (kt_total + ks - 1) / ks;
      if (ks > 1 && ktps < 8) break;
      const long long units = (long long)((n16 + rtw - 1) / rtw) * ks;
      const long long rounds = (units + CUS - 1) / CUS;
      const double per_unit = rtw * ktps * 1024.0 + 0.25 * ktps * 4096.0;
      const double partial = ks > 1 ? 3.0 * 2.0 * ks * (double)m * n16 * 16 * 4 / CUS : 0.0;
      const double cost = rounds * per_unit + partial;
      if (cost < best * 0.999) { best = cost; br = rtw; bk = ks; }
    }
  }
  *rtw_out = br;
  *ks_out = bk;
}

}  // namespace

namespace {

// Checks shared by the decode-projection entry points: rows, shape, x layout and stride, alignment,
// the weight's row tiles per workgroup.
int check_operands(const void* x, long long ldx, int x_tiled, int m, const void* w_tiled, int n, int k, int rtw,
                   const char* who) {
  if (!x || !w_tiled) return fail(PALU_EINVAL, "%s: a required pointer is null", who);
  if (m < 1 || m > 64) return fail(PALU_EINVAL, "%s: rows m = %d must be in 1..64", who, m);
  if (n <= 0 || n % 16) return fail(PALU_EINVAL, "%s: columns n = %d must be a positive multiple of 16", who, n);
  if (k <= 0 || k % 32) return fail(PALU_EINVAL, "%s: k = %d must be a positive multiple of 32", who, k);
  if (x_tiled != 0 && x_tiled != 1) return fail(PALU_EINVAL, "%s: x_tiled = %d must be 0 or 1", who, x_tiled);
  if (!x_tiled && (ldx < k || ldx % 8))
    return fail(PALU_EINVAL, "%s: row stride ldx = %lld must be >= k and a multiple of 8", who, ldx);
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_tiled)) & 15)
    return fail(PALU_EINVAL, "%s: x and w_tiled must be 16-byte aligned", who);
  if (rtw < 1 || rtw > LIN_MAX_RTW)
    return fail(PALU_EINVAL, "%s: rtw = %d (1..%d, as the weight was tiled)", who, rtw, LIN_MAX_RTW);
  return PALU_OK;
}

int launched(hipError_t e, const char* who) {
  if (e != hipSuccess) return fail(PALU_EHIP, "%s launch: %s", who, hipGetErrorString(e));
  return PALU_OK;
}

}  // namespace

extern "C" int palu_linear_plan(int m, int n, int k, int* rtw, int* ks) {
  return palu_linear_plan_ks(m, n, k, 16, rtw, ks);
}

extern "C" int palu_linear_plan_ks(int m, int n, int k, int max_ks, int* rtw, int* ks) {
  palu::g_err[0] = 0;
  if (!rtw || !ks) return fail(PALU_EINVAL, "palu_linear_plan: null output pointer");
  if (m < 1 || m > 64 || n <= 0 || n % 16 || k <= 0 || k % 32 || max_ks < 1)
    return fail(PALU_EINVAL, "palu_linear_plan: m = %d (1..64), n = %d (multiple of 16), k = %d (multiple of 32), max_ks = %d (>= 1)",
                m, n, k, max_ks);
  plan(m, n / 16, k / 32, max_ks, rtw, ks);
  return PALU_OK;
}

extern "C" size_t palu_linear_workspace_bytes(int m, int n, int k, int ks) {
  if (m < 1 || m > 64 || n <= 0 || n % 16 || k <= 0 || k % 32 || ks < 1) return 0;
  return ks > 1 ? (size_t)ks * m * n * sizeof(float) : 0;
}

extern "C" int palu_linear_tiled(const void* x, long long ldx, int x_tiled, int m, const void* w_tiled, int n, int k,
                                 void* y, long long ldy, int y_mode, int rtw, int ks, void* ws, size_t ws_bytes,
                                 hipStream_t stream) {
  palu::g_err[0] = 0;
  const char* who = "palu_linear_tiled";
  if (!y) return fail(PALU_EINVAL, "%s: a required pointer is null", who);
  if (int rc = check_operands(x, ldx, x_tiled, m, w_tiled, n, k, rtw, who)) return rc;
  if (y_mode < PALU_LINEAR_BF16 || y_mode > PALU_LINEAR_SWIGLU_TILED)
    return fail(PALU_EINVAL, "%s: y_mode = %d is not a PALU_LINEAR_* mode", who, y_mode);
  if (y_mode == PALU_LINEAR_BF16 && (ldy < n || ldy % 4))
    return fail(PALU_EINVAL, "%s: row stride ldy = %lld must be >= n and a multiple of 4", who, ldy);
  if (reinterpret_cast<uintptr_t>(y) & (y_mode == PALU_LINEAR_F32_PARTIALS ? 15 : 7))
    return fail(PALU_EINVAL, "%s: y is misaligned for its mode", who);
  if (ks < 1 || ks > 64) return fail(PALU_EINVAL, "%s: ks = %d (1..64)", who, ks);
  if (y_mode == PALU_LINEAR_SWIGLU_TILED && (ks != 1 || n % 64))
    return fail(PALU_EINVAL, "%s: the SwiGLU mode needs ks = 1 and n a multiple of 64, got ks = %d, n = %d", who, ks, n);
  const int n16 = n / 16, kt_total = k / 32;
  const int ktps = (kt_total + ks - 1) / ks;
  if ((long long)((n16 + rtw - 1) / rtw) * ks > 2147483647LL) return fail(PALU_EUNSUPPORTED, "%s: grid too large", who);
  float* part = nullptr;
  if (y_mode == PALU_LINEAR_F32_PARTIALS) {
    part = static_cast<float*>(y);
  } else if (ks > 1) {
    const size_t need = palu_linear_workspace_bytes(m, n, k, ks);
    if (!ws || ws_bytes < need || (reinterpret_cast<uintptr_t>(ws) & 15))
      return fail(PALU_EINVAL, "%s: workspace of %zu bytes (16-byte aligned) needed for %d k slices, got %zu", who,
                  need, ks, ws_bytes);
    part = static_cast<float*>(ws);
  }
  const auto* xb = static_cast<const __bf16*>(x);
  const auto* wb = static_cast<const __bf16*>(w_tiled);
  auto* yb = static_cast<__bf16*>(y);
  const LinEpi ep{};
  const hipError_t e =
      y_mode == PALU_LINEAR_SWIGLU_TILED
          ? launch_epi<EPI_SWIGLU>(x_tiled, rtw, xb, ldx, m, wb, n16, kt_total, ks, ktps, yb, ldy, nullptr, ep, stream)
          : launch_epi<EPI_OUT>(x_tiled, rtw, xb, ldx, m, wb, n16, kt_total, ks, ktps, yb, ldy, part, ep, stream);
  if (int rc = launched(e, who)) return rc;
  if (y_mode == PALU_LINEAR_BF16 && ks > 1) {
    const long long quads = (long long)m * (n / 4);
    const int blocks = (int)std::min<long long>((quads + 255) / 256, 1024);
    hipLaunchKernelGGL(palu_linear_reduce_kernel, dim3(blocks), dim3(256), 0, stream, part, ks, m, n, yb, ldy);
    if (int rc = launched(hipGetLastError(), "palu_linear_tiled reduce")) return rc;
  }
  return PALU_OK;
}

extern "C" size_t palu_linear_argmax_workspace_bytes(int m, int n) {
  if (m < 1 || m > 64 || n <= 0 || n % 16) return 0;
  return (size_t)m * (n / 16) * sizeof(unsigned long long);
}

extern "C" int palu_linear_argmax(const void* x, long long ldx, int x_tiled, int m, const void* w_tiled, int n, int k,
                                  int rtw, int64_t* ids, void* ws, size_t ws_bytes, hipStream_t stream) {
  palu::g_err[0] = 0;
  const char* who = "palu_linear_argmax";
  if (!ids) return fail(PALU_EINVAL, "%s: a required pointer is null", who);
  if (int rc = check_operands(x, ldx, x_tiled, m, w_tiled, n, k, rtw, who)) return rc;
  if (reinterpret_cast<uintptr_t>(ids) & 7) return fail(PALU_EINVAL, "%s: ids must be 8-byte aligned", who);
  const size_t need = palu_linear_argmax_workspace_bytes(m, n);
  if (!ws || ws_bytes < need || (reinterpret_cast<uintptr_t>(ws) & 15))
    return fail(PALU_EINVAL, "%s: workspace of %zu bytes (16-byte aligned) needed, got %zu", who, need, ws_bytes);
  const auto* xb = static_cast<const __bf16*>(x);
  const auto* wb = static_cast<const __bf16*>(w_tiled);
  auto* keys = static_cast<unsigned long long*>(ws);
  auto* out = reinterpret_cast<long long*>(ids);
  return launched(x_tiled ? launch_argmax<true>(rtw, xb, ldx, m, wb, n / 16, k / 32, keys, out, stream)
                          : launch_argmax<false>(rtw, xb, ldx, m, wb, n / 16, k / 32, keys, out, stream),
                  who);
}

extern "C" int palu_linear_swiglu_rmsnorm(const void* x, long long ldx, int x_tiled, int m, const void* w_tiled, int n,
                                          int k, int rtw, float eps, void* y_tiled, hipStream_t stream) {
  palu::g_err[0] = 0;
  const char* who = "palu_linear_swiglu_rmsnorm";
  if (!y_tiled) return fail(PALU_EINVAL, "%s: a required pointer is null", who);
  if (int rc = check_operands(x, ldx, x_tiled, m, w_tiled, n, k, rtw, who)) return rc;
  if (n % 64) return fail(PALU_EINVAL, "%s: n = %d must be a multiple of 64 (gate and up rows interleaved)", who, n);
  if (!(eps >= 0.f)) return fail(PALU_EINVAL, "%s: eps must be >= 0", who);
  if (reinterpret_cast<uintptr_t>(y_tiled) & 15) return fail(PALU_EINVAL, "%s: y_tiled must be 16-byte aligned", who);
  LinEpi ep{};
  ep.eps = eps;
  ep.inv_k = 1.f / (float)k;
  return launched(launch_epi<EPI_SWIGLU_NORM>(x_tiled, rtw, static_cast<const __bf16*>(x), ldx, m,
                                              static_cast<const __bf16*>(w_tiled), n / 16, k / 32, 1, k / 32,
                                              static_cast<__bf16*>(y_tiled), 0, nullptr, ep, stream),
                  who);
}

extern "C" int palu_linear_residual(const void* x, long long ldx, int x_tiled, int m, const void* w_tiled, int n, int k,
                                    int rtw, void* h, long long ldh, void* h_tiled, hipStream_t stream) {
  palu::g_err[0] = 0;
  const char* who = "palu_linear_residual";
  if (!h) return fail(PALU_EINVAL, "%s: a required pointer is null", who);
  if (int rc = check_operands(x, ldx, x_tiled, m, w_tiled, n, k, rtw, who)) return rc;
  if (ldh < n || ldh % 4 || (reinterpret_cast<uintptr_t>(h) & 7))
    return fail(PALU_EINVAL, "%s: h must be 8-byte aligned with a row stride ldh = %lld >= n and a multiple of 4", who,
                ldh);
  if (h_tiled && (n % 32 || (reinterpret_cast<uintptr_t>(h_tiled) & 15)))
    return fail(PALU_EINVAL, "%s: a tiled copy of h needs n = %d a multiple of 32 and 16-byte alignment", who, n);
  LinEpi ep{};
  ep.h = static_cast<__bf16*>(h);
  ep.ldh = ldh;
  ep.h_tiled = static_cast<__bf16*>(h_tiled);
  return launched(launch_epi<EPI_RESID>(x_tiled, rtw, static_cast<const __bf16*>(x), ldx, m,
                                        static_cast<const __bf16*>(w_tiled), n / 16, k / 32, 1, k / 32, nullptr, 0,
                                        nullptr, ep, stream),
                  who);
}

extern "C" int palu_linear_qkv(const void* x, long long ldx, int x_tiled, int m, const void* w_tiled, int n, int k,
                               int rtw, const int32_t* pos, const float* cos_table, const float* sin_table,
                               int table_rows, int n_heads, void* q_out, void* k_cache, int k_layout, int k_col_offset,
                               int k_group_stride, int k_width, int k_rope, void* v_cache, int v_layout,
                               int v_col_offset, int v_group_stride, int v_width, int n_groups, int seq_len,
                               hipStream_t stream) {
  palu::g_err[0] = 0;
  const char* who = "palu_linear_qkv";
  if (int rc = check_operands(x, ldx, x_tiled, m, w_tiled, n, k, rtw, who)) return rc;
  LinEpi ep{};
  ep.q = QkvEpi{pos, cos_table, sin_table, table_rows, n_heads, static_cast<__bf16*>(q_out),
                static_cast<__bf16*>(k_cache), k_layout, k_col_offset, k_group_stride, k_width, k_rope ? 1 : 0,
                static_cast<__bf16*>(v_cache), v_layout, v_col_offset, v_group_stride, v_width, n_groups, seq_len};
  if (int rc = check_qkv_epi(ep.q, m, n, x, who)) return rc;
  // Each output column must belong to at most one part of the row: q heads first, then K and V slices
  // that neither overlap the q heads, each other, nor (with several groups) their neighbours.
  const long long q_end = (long long)n_heads * HD;
  const long long k_end = (long long)k_col_offset + (long long)(n_groups - 1) * k_group_stride + k_width;
  const long long v_end = (long long)v_col_offset + (long long)(n_groups - 1) * v_group_stride + v_width;
  if (k_col_offset < q_end || v_col_offset < q_end || (k_col_offset < v_end && v_col_offset < k_end) ||
      (n_groups > 1 && (k_group_stride < k_width || v_group_stride < v_width)))
    return fail(PALU_EINVAL, "%s: the q, K and V column ranges (and the groups' slices) must not overlap", who);
  return launched(launch_epi<EPI_QKV>(x_tiled, rtw, static_cast<const __bf16*>(x), ldx, m,
                                      static_cast<const __bf16*>(w_tiled), n / 16, k / 32, 1, k / 32, nullptr, 0,
                                      nullptr, ep, stream),
                  who);
}
