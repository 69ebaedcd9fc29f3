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
// Outputs (y_mode): bf16 y [m][n] (split partials summed by a second launch); the fp32 split partials
// [KS][m][n] themselves, for a consumer that sums them (palu_rmsnorm's residual input, palu_qkv_post);
// or, for a gate / up weight interleaved eight rows at a time (tile_weight of
// palu_tt.decoder_ops.interleave_gate_up), silu(gate) * up in the tiled activation layout.
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

constexpr int LIN_NW = 4;
constexpr int LIN_MT = 4;                       // 16-row activation tiles: m <= 64
constexpr int LIN_MAX_RTW = 8;

template <int RTW>
struct LinSmem {
  static constexpr int SLOT = RTW * LIN_MT * 64;          // f32x4 per wave partial
  static constexpr int BYTES = LIN_NW * SLOT * 16;        // every wave's partial
};

// NB register buffers per wave, so each step's loads are issued NB - 1 steps before its MFMAs. Weight
// and activation tiles of one step share a buffer: loads return in issue order, so an activation tile
// loaded later than the weights would make every wait a wait for those weights too.
template <int RTW, int NB, bool XT, bool SWIGLU>
__global__ __launch_bounds__(LIN_NW * 64) void palu_linear_kernel(const __bf16* __restrict__ x, long long ldx, int m,
                                                                  const __bf16* __restrict__ wt, int n16, int kt_total,
                                                                  int ks_count, int kt_per_split,
                                                                  __bf16* __restrict__ y, long long ldy,
                                                                  float* __restrict__ part) {
  using SM = LinSmem<RTW>;
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

  // Every load is issued on every path (row tiles past rt_cnt read the last row tile, k tiles past the
  // slice read the matrix's last k tile; their products are never stored), so each wait in the loop is
  // for exactly the loads of the buffer about to be used.
  bf16x8 wa[NB][RTW], xb[NB][LIN_MT];
  auto load = [&](int buf, int kt) {
    kt = min(kt, kt_total - 1);
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
  };

  // The loop is unrolled by NB so that buffer indices are compile-time, and has no branch: steps past the
  // wave's count (the rest of the last round) load clamped tiles and multiply them by zero activations.
  // The scheduling barriers keep each step's loads ahead of the earlier step's MFMAs (left alone, the
  // compiler sinks every load to its first use and the wave has one tile in flight).
  const int kt0 = kt_lo + w;
  const int nsteps = kt0 < kt_hi ? (kt_hi - kt0 + LIN_NW - 1) / LIN_NW : 0;   // uniform per wave
#pragma unroll
  for (int j = 0; j < NB - 1; ++j) load(j, kt0 + j * LIN_NW);
  for (int s = 0; s < nsteps; s += NB) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      load((j + NB - 1) % NB, kt0 + (s + j + NB - 1) * LIN_NW);
      __builtin_amdgcn_sched_barrier(0);
      compute(j, s + j < nsteps);
    }
  }

  // The waves' partials meet in LDS (slot layout [wave][r][mt][lane] of f32x4); each wave then sums
  // the four slots of every fourth (r, mt) tile and stores that tile, so the epilogue's arithmetic and
  // stores are spread over the four SIMDs.
#pragma unroll
  for (int r = 0; r < RTW; ++r)
#pragma unroll
    for (int mt = 0; mt < LIN_MT; ++mt) red[w * SM::SLOT + (r * LIN_MT + mt) * 64 + lane] = acc[r][mt];
  __syncthreads();

  // Lane (g, mm) of tile (r, mt) holds y^T[16 (rt0 + r) + 4 g + i][16 mt + mm], i < 4: four consecutive
  // output columns of activation row 16 mt + mm.
#pragma unroll
  for (int t = 0; t < RTW * LIN_MT; ++t) {
    if (t % LIN_NW != w) continue;                         // uniform per wave
    const int r = t / LIN_MT, mt = t % LIN_MT;
    f32x4 v = red[(r * LIN_MT + mt) * 64 + lane];
#pragma unroll
    for (int q = 1; q < LIN_NW; ++q) v += red[q * SM::SLOT + (r * LIN_MT + mt) * 64 + lane];
    const int row = 16 * mt + mm;
    if constexpr (SWIGLU) {
      // Gate / up pairs: rows 0-7 of row tile rt are gate columns 8 rt .. 8 rt + 7 and rows 8-15 the up
      // columns of the same outputs (tile_weight of the interleaved weight), so lane (g, mm) with g < 2
      // holds gate columns 8 rt + 4 g + i and lane (g + 2, mm), 32 lanes on, the matching up values.
      // out = silu(gate) * up, stored in the tiled activation layout (64 rows x n / 2) the next
      // projection reads.
      f32x4 up;
#pragma unroll
      for (int i = 0; i < 4; ++i) up[i] = __shfl_xor(v[i], 32, 64);
      if (g >= 2 || row >= m || r >= rt_cnt) continue;
      const int col = 8 * (rt0 + r) + 4 * g;
      bf16x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = (__bf16)((v[i] / (1.f + __expf(-v[i]))) * up[i]);
      const long long off = ((long long)((col >> 5) * 4 + (row >> 4)) * 64 + 16 * ((col & 31) >> 3) + (row & 15)) * 8
                            + (col & 7);
      *reinterpret_cast<bf16x4*>(y + off) = o;
    } else {
      if (row >= m || r >= rt_cnt) continue;
      const long long col = 16LL * (rt0 + r) + 4 * g;
      if (part) {
        *reinterpret_cast<f32x4*>(part + ((long long)ks * m + row) * (16LL * n16) + col) = v;
      } else {
        bf16x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = (__bf16)v[i];
        *reinterpret_cast<bf16x4*>(y + row * ldy + col) = o;
      }
    }
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

template <int RTW, bool XT, bool SWIGLU>
hipError_t launch_cfg(const __bf16* x, long long ldx, int m, const __bf16* wt, int n16, int kt_total, int ks,
                      int ktps, __bf16* y, long long ldy, float* part, hipStream_t s) {
  constexpr int NB = RTW <= 2 ? 8 : 4;                    // about 8 KB of weights in flight per wave
  auto kern = palu_linear_kernel<RTW, NB, XT, SWIGLU>;
  constexpr int lds = LinSmem<RTW>::BYTES;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int groups = (n16 + RTW - 1) / RTW;
  hipLaunchKernelGGL(kern, dim3(groups * ks), dim3(LIN_NW * 64), lds, s, x, ldx, m, wt, n16, kt_total, ks, ktps, y,
                     ldy, part);
  return hipGetLastError();
}

template <bool XT, bool SWIGLU>
hipError_t launch_rtw(int rtw, const __bf16* x, long long ldx, int m, const __bf16* wt, int n16, int kt_total, int ks,
                      int ktps, __bf16* y, long long ldy, float* part, hipStream_t s) {
  switch (rtw) {
    case 1: return launch_cfg<1, XT, SWIGLU>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, s);
    case 2: return launch_cfg<2, XT, SWIGLU>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, s);
    case 3: return launch_cfg<3, XT, SWIGLU>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, s);
    case 4: return launch_cfg<4, XT, SWIGLU>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, s);
    case 5: return launch_cfg<5, XT, SWIGLU>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, s);
    case 6: return launch_cfg<6, XT, SWIGLU>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, s);
    case 7: return launch_cfg<7, XT, SWIGLU>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, s);
    default: return launch_cfg<8, XT, SWIGLU>(x, ldx, m, wt, n16, kt_total, ks, ktps, y, ldy, part, s);
  }
}

// Row tiles per workgroup and k slices: the pair whose busiest CU streams the fewest bytes, counting the
// activation re-reads (4 KB per k tile and workgroup, from L2, weighted at a quarter of a weight byte)
// and the split partials (written and read once in fp32, weighted at three weight bytes each: measured,
// the k-split passes cost more than their bytes).
void plan(int m, int n16, int kt_total, int* rtw_out, int* ks_out) {
  constexpr int CUS = 256;
  double best = 1e300;
  int br = 1, bk = 1;
  for (int rtw = 1; rtw <= LIN_MAX_RTW; ++rtw) {
    for (int ks = 1; ks <= 16; ks *= 2) {
      const int ktps = (kt_total + ks - 1) / ks;
      if (ks > 1 && ktps < 2 * LIN_NW) break;
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

extern "C" int palu_linear_plan(int m, int n, int k, int* rtw, int* ks) {
  palu::g_err[0] = 0;
  if (!rtw || !ks) return fail(PALU_EINVAL, "palu_linear_plan: null output pointer");
  if (m < 1 || m > 64 || n <= 0 || n % 16 || k <= 0 || k % 32)
    return fail(PALU_EINVAL, "palu_linear_plan: m = %d (1..64), n = %d (multiple of 16), k = %d (multiple of 32)", m, n, k);
  plan(m, n / 16, k / 32, rtw, ks);
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
  if (!x || !w_tiled || !y) return fail(PALU_EINVAL, "palu_linear_tiled: a required pointer is null");
  if (m < 1 || m > 64) return fail(PALU_EINVAL, "palu_linear_tiled: rows m = %d must be in 1..64", m);
  if (n <= 0 || n % 16) return fail(PALU_EINVAL, "palu_linear_tiled: columns n = %d must be a positive multiple of 16", n);
  if (k <= 0 || k % 32) return fail(PALU_EINVAL, "palu_linear_tiled: k = %d must be a positive multiple of 32", k);
  if (x_tiled != 0 && x_tiled != 1) return fail(PALU_EINVAL, "palu_linear_tiled: x_tiled = %d must be 0 or 1", x_tiled);
  if (y_mode < PALU_LINEAR_BF16 || y_mode > PALU_LINEAR_SWIGLU_TILED)
    return fail(PALU_EINVAL, "palu_linear_tiled: y_mode = %d is not a PALU_LINEAR_* mode", y_mode);
  if (!x_tiled && (ldx < k || ldx % 8))
    return fail(PALU_EINVAL, "palu_linear_tiled: row stride ldx = %lld must be >= k and a multiple of 8", ldx);
  if (y_mode == PALU_LINEAR_BF16 && (ldy < n || ldy % 4))
    return fail(PALU_EINVAL, "palu_linear_tiled: row stride ldy = %lld must be >= n and a multiple of 4", ldy);
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_tiled)) & 15)
    return fail(PALU_EINVAL, "palu_linear_tiled: x and w_tiled must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(y) & (y_mode == PALU_LINEAR_F32_PARTIALS ? 15 : 7))
    return fail(PALU_EINVAL, "palu_linear_tiled: y is misaligned for its mode");
  if (rtw < 1 || rtw > LIN_MAX_RTW || ks < 1 || ks > 64)
    return fail(PALU_EINVAL, "palu_linear_tiled: rtw = %d (1..%d, as the weight was tiled) and ks = %d (1..64)", rtw,
                LIN_MAX_RTW, ks);
  if (y_mode == PALU_LINEAR_SWIGLU_TILED && (ks != 1 || n % 64))
    return fail(PALU_EINVAL, "palu_linear_tiled: the SwiGLU mode needs ks = 1 and n a multiple of 64, got ks = %d, n = %d",
                ks, n);
  const int n16 = n / 16, kt_total = k / 32;
  const int ktps = (kt_total + ks - 1) / ks;
  if ((long long)((n16 + rtw - 1) / rtw) * ks > 2147483647LL) return fail(PALU_EUNSUPPORTED, "palu_linear_tiled: grid too large");
  float* part = nullptr;
  if (y_mode == PALU_LINEAR_F32_PARTIALS) {
    part = static_cast<float*>(y);
  } else if (ks > 1) {
    const size_t need = palu_linear_workspace_bytes(m, n, k, ks);
    if (!ws || ws_bytes < need || (reinterpret_cast<uintptr_t>(ws) & 15))
      return fail(PALU_EINVAL, "palu_linear_tiled: workspace of %zu bytes (16-byte aligned) needed for %d k slices, got %zu",
                  need, ks, ws_bytes);
    part = static_cast<float*>(ws);
  }
  const auto* xb = static_cast<const __bf16*>(x);
  const auto* wb = static_cast<const __bf16*>(w_tiled);
  auto* yb = static_cast<__bf16*>(y);
  hipError_t e;
  if (y_mode == PALU_LINEAR_SWIGLU_TILED)
    e = x_tiled ? launch_rtw<true, true>(rtw, xb, ldx, m, wb, n16, kt_total, ks, ktps, yb, ldy, nullptr, stream)
                : launch_rtw<false, true>(rtw, xb, ldx, m, wb, n16, kt_total, ks, ktps, yb, ldy, nullptr, stream);
  else
    e = x_tiled ? launch_rtw<true, false>(rtw, xb, ldx, m, wb, n16, kt_total, ks, ktps, yb, ldy, part, stream)
                : launch_rtw<false, false>(rtw, xb, ldx, m, wb, n16, kt_total, ks, ktps, yb, ldy, part, stream);
  if (e != hipSuccess) return fail(PALU_EHIP, "palu_linear_tiled launch: %s", hipGetErrorString(e));
  if (y_mode == PALU_LINEAR_BF16 && ks > 1) {
    const long long quads = (long long)m * (n / 4);
    const int blocks = (int)std::min<long long>((quads + 255) / 256, 1024);
    hipLaunchKernelGGL(palu_linear_reduce_kernel, dim3(blocks), dim3(256), 0, stream, part, ks, m, n, yb, ldy);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(PALU_EHIP, "palu_linear_tiled reduce launch: %s", hipGetErrorString(e));
  }
  return PALU_OK;
}
