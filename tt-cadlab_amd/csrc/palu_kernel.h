// Palu fused latent flash-decode for MI355X (gfx950): the decode kernels, shared by the translation
// units that instantiate them (palu_decode_*.hip) and the C-ABI (palu_capi.hip).
//
// One work item is one (batch row b, KV head h). Per position p <= cur_pos[b] the item's key is
// rebuilt from its latent row, K[p] = RoPE_p(lat_k[p] @ u_k[h]), and the GQA group of query heads
// that share KV head h runs an online-softmax flash-decode over those keys. With the absorbed-V
// layout the value rows are the V latent itself, so the output is [B, n_q, r_v] in latent space
// (the up-projection lives in wo_fused). Semantics follow the reference op
// ttnn.transformer.palu_sdpa_decode (docs/superpowers/specs/2026-09-10-palu-tt-stage2-design.md:47-81,
// fp32 model palu_tt/fused.py:82-107).
//
// Kernel shape (MFMA work is v_mfma_f32_16x16x32_bf16 for the K rebuild and PV, _f16 for QK against
// the fp16 rotated K; fp32 accumulate):
//   * A workgroup owns one item and one split of its sequence. Its NW waves take pairs of 32-position
//     blocks from an LDS counter (or, in deterministic mode, every NW-th pair) and stream each block
//     from HBM straight into registers, the next block's loads in flight while the current one is
//     computed. The block index lives in a scalar register and every load is issued on every path,
//     so the compiler waits on exactly the loads a step consumes.
//   * Two cache layouts. ROWS is the reference's logical [B, G, S, r] row-major tensor. TILED stores
//     every 32-position block as r / 16 tiles of 1 KB already in MFMA operand order (K-tile order for
//     K, V-tile order for V; see include/palu_mi355x.h), so each wave load instruction is one
//     contiguous 1 KB, issued nontemporal (the stream is read once per decode step).
//   * K is rebuilt transposed, K^T[d][p] = u_k^T[d][:] . lat[p][:], one 32-dim slice at a time: the
//     accumulator layout gives every lane one position and 4 consecutive head dims per 16-dim tile, so
//     each RoPE pair (Meta-interleaved dims 2f, 2f+1) sits in one lane and the rotation is plain VALU
//     work: each fp32 accumulator pair is converted to fp16 (round toward zero, saturating) and
//     rotated with packed fp16 multiplies.
//   * RoPE is applied pair-relative: K rows are rotated by their offset t < 64 inside a pair of
//     blocks (an LDS table in lane order), and the query is rotated back by the pair base once per
//     pair, q~ = R_{-base} q, with cos/sin of the base built by angle addition from two small LDS
//     tables (base = 1024 H + 64 Lo). Rotations in one plane commute, so q~ . R_t k = q . R_{base+t} k,
//     the score of the reference.
//   * The rotated fp16 K slice is the A operand of the QK MFMA as it stands; the head dim is
//     contracted in a permuted order that the query operand mirrors, so no lane shuffles are needed.
//   * Scores come out with one head per lane column. The online softmax runs in the exp2 domain
//     (scale * log2 e folded into q~) with a lazily refreshed running max, and the probabilities feed
//     the PV MFMA directly as its B operand. TILED V is already the PV A operand; ROWS V is regrouped
//     by an MFMA against an identity tile (exact in bf16).
//   * The waves of a workgroup merge their (O, m, l) partials in LDS. When B * n_kv is not a whole
//     number of chip-fills, items are cut into length-aware chunks (planned on the device from
//     cur_pos) and the chunks of one item are merged by a second small kernel through a
//     caller-provided workspace.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <math.h>
#include <stdio.h>
#include <stdarg.h>
#include <string.h>
#include <type_traits>

#include "../../include/palu_mi355x.h"

namespace palu {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int HD = 128;     // head dim
constexpr int MAX_GROUPS = 32;  // latent groups per layer of the grouped-latent (u_v) kernels
constexpr int BLK = 32;     // positions per block: two 16-position MFMA tiles, also the rotation chunk
constexpr float NEG_INF = -__builtin_huge_valf();
constexpr float LAZY_RESCALE_LOG2 = 8.0f;  // running max is refreshed when a score exceeds it by > 2^8

struct DecodeArgs {
  const __bf16* q;        // [B, n_q, HD], already rotated at its own position
  const __bf16* k;        // latent [B, n_groups, S, RK]   or full rotated K [B, n_kv, S, HD]
  const __bf16* v;        // latent [B, n_groups, S, RV]   or full V [B, n_kv, S, RV]
  const __bf16* w_rot;    // [n_kv, RK, 2*HD]; columns 0..HD-1 are u_k (Meta head order)
  const void* cs;         // [cs_rows, 2*HD]: [cos | sin], Meta-interleaved, fp32 or bf16
  const int32_t* cur_pos; // [B], inclusive last valid position
  void* out;              // [B, n_q, RV]
  float* ws;              // split partials: [n_wg, 16, RV + 2] (M-LRD / stock), see glrd for its own
  size_t ws_bytes;
  long long k_sb, k_sg;   // element strides of k: batch, group (row stride is RK / HD)
  long long v_sb, v_sg;
  int B, n_q, n_kv, rep, hpg, S, cs_rows;
  int split_len;          // grouped-latent kernels: positions per workgroup split, a multiple of BLK
  int n_splits;
  int n_wg;               // M-LRD / stock decode: workgroups launched; n_wg > B * n_kv splits items by length
  int balanced;           // 1 when n_wg > B * n_kv (length-aware chunks, merged through ws)
  unsigned long long epoch;  // balanced: this call's tag for the items' chunk counters (CHUNK_TAG | call number)
  int deterministic;      // 1: wave w takes blocks w, w + NW, ... (reproducible); 0: blocks from a counter
  int out_tiled;          // 1: out in the 64-row tiled activation layout of the next projection (B <= 64)
  int grouped_streams;    // grouped latents stored compactly, each group at its own ranks (PALU_LAYOUT_TILED_GROUPED)
  float qscale;           // softmax scale * log2(e)
  // Paged caches: k/v are page pools [n_pages, G, page_size, width] (rows or tiled) and k_sb / v_sb are
  // page strides; the page of block J of row b is page_table[b * pt_stride + (J >> page_shift)].
  const int32_t* page_table;
  int pt_stride, n_pages, page_shift;
  // Grouped latents with in-kernel V (u_v given): [n_kv, RV, HD] per KV head; k/v are then the group
  // latents [B, n_groups, S, RK / RV] in the tiled layout, and the output is HD wide.
  const __bf16* u_v;
  int rk, rv;             // latent widths of the caches (the grouped-latent kernels take them at run time)
  // Grouped latents: each group's own ranks (<= rk / rv, multiples of 32; the cache columns past them
  // are never read), and the groups one scores launch covers (grp_lo .. grp_lo + grp_cnt - 1, whose
  // K rank is rk_eff).
  short grk[MAX_GROUPS], grv[MAX_GROUPS];
  int grp_lo, grp_cnt, rk_eff;
  // Grouped-latent streams: group g of row b starts at element b * k_sb + gko[g] and is gkw[g] wide (the
  // padded layout: g * k_sg and rk; the compact one: S times the widths of the groups before it, and
  // the group's own rank). Same for V.
  long long gko[MAX_GROUPS], gvo[MAX_GROUPS];
  short gkw[MAX_GROUPS], gvw[MAX_GROUPS];
  // Grouped-latent PV plan, per group: gns2 splits of gsl2 positions; its workgroups are gwg2[g] ..
  // gwg2[g + 1] - 1 and its partial rows start at gprow[g] ([row][head of the group][split] order).
  short gns2[MAX_GROUPS];
  int gsl2[MAX_GROUPS], gwg2[MAX_GROUPS + 1], gprow[MAX_GROUPS];
};

// Error reporting (defined in palu_capi.hip): formats the message for palu_last_error, returns code.
int fail(int code, const char* fmt, ...);
extern thread_local char g_err[1024];

// Last-finisher counters (count_done; the chunks of split decode items): bits 63..48 a fixed tag,
// 47..16 the call number (next_epoch, one per launch that counts), 15..0 the count so far.
constexpr unsigned long long CHUNK_TAG = 0xA5C3ull << 48;
unsigned long long next_epoch();   // defined in palu_capi.hip

// The decode step's QKV epilogue (palu_qkv_post over split partials, palu_linear_qkv inside the
// projection): where each part of a QKV output row goes. q heads are columns h * 128 .. of the row,
// rotated at pos[b] into q_out [B, nh, 128]; group g's K slice is columns k_off + g * k_gs, k_w wide
// (rotated too when k_rope: the stock path's full-rank K, one head per group), appended at pos[b] to
// the K cache (layout k_layout); V the same with v_*. Caches are [B, G, S, width] streams.
struct QkvEpi {
  const int32_t* pos;
  const float* cos_t;
  const float* sin_t;
  int table_rows, nh;
  __bf16* q_out;
  __bf16* kc;
  int k_layout, k_off, k_gs, k_w, k_rope;
  __bf16* vc;
  int v_layout, v_off, v_gs, v_w;
  int G, S;
};

// Checks a QkvEpi for a QKV output of `batch` rows of `ncols` columns read from src (defined in
// palu_capi.hip; `who` names the entry point in the message).
int check_qkv_epi(const QkvEpi& e, int batch, int ncols, const void* src, const char* who);

// Waves per workgroup: 8 (two per SIMD) where the kernel fits 256 registers, else 4 (one per SIMD,
// which lets the compiler use the full 512-entry register file instead of spilling).
template <int RK, int RV, bool KFULL, bool TILED>
constexpr int pick_nw() {
  // 8 waves where the kernel fits 256 VGPRs without spilling (checked per instantiation and layout with
  // -Rpass-analysis=kernel-resource-usage: every latent width pair but r_k 64 / r_v 128 does), else 4
  // waves with the 512-register budget.
  if (KFULL) return 8;
  return ((RK + 31) / 32 == 2 && RV == 128) ? 4 : 8;   // r_k 48 holds the registers of r_k 64
}
constexpr int MIN_NW = 4;
constexpr int TARGET_WGS = 256;  // one workgroup per CU at full occupancy of the chip

struct Plan {
  int n_splits, split_len;
};

inline Plan plan_splits(int items, int S, int nw) {
  // Positions per workgroup: about TARGET_WGS workgroups over the whole job, in whole blocks for
  // every wave; a sequence is split across workgroups only when its items alone cannot fill the chip.
  const long long total = (long long)items * S;
  const long long unit = (long long)BLK * nw;
  long long per_wg = (total + TARGET_WGS - 1) / TARGET_WGS;
  per_wg = ((per_wg + unit - 1) / unit) * unit;
  const long long whole = (((long long)S + BLK - 1) / BLK) * BLK;
  if (per_wg > whole) per_wg = whole;
  return Plan{(int)((S + per_wg - 1) / per_wg), (int)per_wg};
}

inline size_t ws_bytes(int items, int n_splits, int rv) {
  return n_splits <= 1 ? 0 : (size_t)items * n_splits * 16 * (rv + 2) * sizeof(float);
}

// M-LRD / stock decode: workgroups per launch, a whole number of chip-fills of TARGET_WGS. When the
// work items fill it exactly, each workgroup owns one item; otherwise items are cut into chunks by
// their actual lengths (device side, from cur_pos) and the partials of the split ones are merged.
inline int decode_workgroups(int items) { return ((items + TARGET_WGS - 1) / TARGET_WGS) * TARGET_WGS; }
inline size_t decode_ws_bytes(int items, int rv) {
  const int wg = decode_workgroups(items);
  // partial slots [wg][16][rv + 2] floats, then one 8-byte chunk counter per item
  return wg == items ? 0 : (size_t)wg * 16 * (rv + 2) * sizeof(float) + (size_t)items * sizeof(unsigned long long);
}


// Decode dispatchers, one translation unit each (cs_dtype / out_dtype are PALU_DTYPE_*).
int dispatch_latent_rows(const DecodeArgs& a, int rk, int rv, int cs_dtype, int out_dtype, hipStream_t s);
int dispatch_latent_tiled(const DecodeArgs& a, int rk, int rv, int cs_dtype, int out_dtype, hipStream_t s);
int dispatch_latent_rows_paged(const DecodeArgs& a, int rk, int rv, int cs_dtype, int out_dtype, hipStream_t s);
int dispatch_latent_tiled_paged(const DecodeArgs& a, int rk, int rv, int cs_dtype, int out_dtype, hipStream_t s);
// tiled caches whose K width is an odd multiple of 16 (48, 80, 112)
int dispatch_latent_tiled_k16(const DecodeArgs& a, int rk, int rv, int cs_dtype, int out_dtype, hipStream_t s);
int dispatch_latent_tiled_paged_k16(const DecodeArgs& a, int rk, int rv, int cs_dtype, int out_dtype, hipStream_t s);
int dispatch_full(const DecodeArgs& a, bool tiled, bool paged, int dv, bool f32_out, hipStream_t s);
int dispatch_glrd(const DecodeArgs& a, bool rows, int cs_dtype, int out_dtype, hipStream_t s);
size_t glrd_workspace_bytes(int batch, int n_q, int n_kv, int n_groups, int seq_len, int r_v);

}  // namespace palu

// Kernels and launch templates are local to each translation unit that instantiates them.
namespace {

using namespace palu;

// Offset (elements) of width-index k of position p inside one (b, g) stream of width R, K-tile order.
// A block's positions t = p % 32 with (t / 4) % 2 == c form half-block c, 16 R elements from c * 16 R:
// R / 32 full tiles of 512 (lane 16 gg + nn holds width-indices 32 kb + 8 gg .. +7), then, when R is an
// odd multiple of 16, one half tile of 256 (lane 16 gg + nn holds width-indices 32 (R / 32) + 4 gg .. +3,
// the low half of its 32-deep MFMA operand); nn = 4 (t / 8) + t % 4 is the position's operand column.
__device__ __forceinline__ long long tiled_k_offset(int p, int k, int R) {
  const int t = p & 31, c = (t >> 2) & 1, nn = ((t >> 3) << 2) | (t & 3);
  const int kb = k >> 5, kbf = R >> 5;
  const long long half = (long long)(p >> 5) * (32 * R) + c * 16 * R;
  if (kb < kbf) return half + (kb * 64 + 16 * ((k >> 3) & 3) + nn) * 8 + (k & 7);
  return half + kbf * 512 + (16 * ((k & 15) >> 2) + nn) * 4 + (k & 3);
}

// Stores width-indices k .. k + 7 (k a multiple of 8) of position p in K-tile order: one 16-byte store
// in a full tile, two 8-byte stores 16 lanes apart in the half tile.
__device__ __forceinline__ void store_k8(__bf16* stream, int p, int k, int R, const bf16x8 x) {
  const long long o = tiled_k_offset(p, k, R);
  if ((k >> 5) < (R >> 5)) {
    *reinterpret_cast<bf16x8*>(stream + o) = x;
  } else {
    *reinterpret_cast<bf16x4*>(stream + o) = bf16x4{x[0], x[1], x[2], x[3]};
    *reinterpret_cast<bf16x4*>(stream + o + 64) = bf16x4{x[4], x[5], x[6], x[7]};
  }
}

// V-tile order: tile mt = k / 16, slot 16 * (t / 8) + k % 16, element t % 8 (t = p % 32).
__device__ __forceinline__ long long tiled_v_offset(int p, int k, int R) {
  const int t = p & 31;
  return (long long)(p >> 5) * (32 * R) + ((k >> 4) * 64 + 16 * (t >> 3) + (k & 15)) * 8 + (t & 7);
}

// Element offset of (row, col) in the 64-row tiled activation layout of the decode projections
// (palu_linear_tiled with x_tiled): tile (col / 32, row / 16) of 1 KB, lane 16 ((col % 32) / 8) + row % 16,
// element col % 8.
__device__ __forceinline__ long long tiled_row_offset(int row, int col) {
  return ((long long)((col >> 5) * 4 + (row >> 4)) * 64 + 16 * ((col & 31) >> 3) + (row & 15)) * 8 + (col & 7);
}

// Meta RoPE of N consecutive fp32 values of one head starting at head column c (even), table row pr:
// pairs (2i, 2i+1) -> (x0 c - x1 s, x1 c + x0 s). The fused multiply-adds are written out so that every
// kernel that rotates rounds the same way.
template <int N>
__device__ __forceinline__ void rope_meta(float (&v)[N], const float* cos_t, const float* sin_t, int pr, int c) {
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const float cs = cos_t[(long long)pr * HD + c + 2 * i], sn = sin_t[(long long)pr * HD + c + 2 * i];
    const float x0 = v[2 * i], x1 = v[2 * i + 1];
    v[2 * i] = fmaf(x0, cs, -(x1 * sn));
    v[2 * i + 1] = fmaf(x1, cs, x0 * sn);
  }
}

// N = 4 or 8 consecutive fp32 values of QKV output row b, starting at a multiple of N inside one part
// of the row: q head gi (kind 0), or group gi's K (kind 1) or V slice (kind 2), at column c of that head
// or slice. Rotated where the epilogue says, rounded to bf16 once, and stored to q_out or appended to
// the cache at the row's position p = pos[b] (positions outside the cache are not appended).
template <int N>
__device__ __forceinline__ void qkv_store(const QkvEpi& e, int b, int p, int kind, int gi, int c, float (&v)[N]) {
  typedef __bf16 bfn __attribute__((ext_vector_type(N)));
  if (kind == 0 || (kind == 1 && e.k_rope)) {
    const int pr = p < 0 ? 0 : (p >= e.table_rows ? e.table_rows - 1 : p);
    rope_meta<N>(v, e.cos_t, e.sin_t, pr, c);
  }
  bfn o;
#pragma unroll
  for (int j = 0; j < N; ++j) o[j] = (__bf16)v[j];
  if (kind == 0) {
    *reinterpret_cast<bfn*>(e.q_out + ((long long)b * e.nh + gi) * HD + c) = o;
    return;
  }
  if (p < 0 || p >= e.S) return;
  const int layout = kind == 1 ? e.k_layout : e.v_layout, width = kind == 1 ? e.k_w : e.v_w;
  __bf16* stream = (kind == 1 ? e.kc : e.vc) + ((long long)b * e.G + gi) * e.S * width;
  if (layout == PALU_LAYOUT_ROWS) {
    *reinterpret_cast<bfn*>(stream + (long long)p * width + c) = o;
  } else if (layout == PALU_LAYOUT_TILED) {
    if constexpr (N == 8) {
      store_k8(stream, p, c, width, o);
    } else {
      *reinterpret_cast<bfn*>(stream + tiled_k_offset(p, c, width)) = o;   // 4 width-indices share a slot
    }
  } else {
    const long long off = tiled_v_offset(p, c, width);   // N slots 16 bytes apart
#pragma unroll
    for (int j = 0; j < N; ++j) stream[off + 8 * j] = o[j];
  }
}

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
// Four bf16 in the low half of an MFMA operand, zeros above: a half K tile's 4 values per lane on the
// 32-deep product, whose upper k slots then contribute exactly 0 (both operands zero there).
__device__ __forceinline__ bf16x8 low4(const bf16x4 h) {
  const bf16x4 z = {};
  return __builtin_shufflevector(h, z, 0, 1, 2, 3, 4, 5, 6, 7);
}

// fp32 pair -> fp16 pair, rounded toward zero: finite inputs beyond the fp16 range saturate to
// +-65504 instead of becoming infinite.
__device__ __forceinline__ f16x2 to_f16x2(float a, float b) {
  return __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(a, b));
}

// max of 8 without NaN canonicalisation (v_maximum3_f32)
__device__ __forceinline__ float max8(f32x4 a, f32x4 b) {
  const float x = __builtin_elementwise_maximum(__builtin_elementwise_maximum(a[0], a[1]), a[2]);
  const float y = __builtin_elementwise_maximum(__builtin_elementwise_maximum(a[3], b[0]), b[1]);
  const float z = __builtin_elementwise_maximum(__builtin_elementwise_maximum(b[2], b[3]), x);
  return __builtin_elementwise_maximum(y, z);
}

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(__bf16 x) { return (float)x; }

// Element index of output (row b, column col) of [B, row_len]: row-major, or the 64-row tiled activation
// layout that palu_linear_tiled reads (tile (col / 32, b / 16) of 1 KB, lane 16 ((col % 32) / 8) + b % 16).
__device__ __forceinline__ long long out_index(const DecodeArgs& a, int b, long long col, long long row_len) {
  if (a.out_tiled)
    return ((long long)((col >> 5) * 4 + (b >> 4)) * 64 + 16 * ((col & 31) >> 3) + (b & 15)) * 8 + (col & 7);
  return (long long)b * row_len + col;
}

__device__ __forceinline__ void store_out(float* p, float v) { *p = v; }
__device__ __forceinline__ void store_out(__bf16* p, float v) { *p = (__bf16)v; }

__device__ __forceinline__ bf16x8 pack8(f32x4 lo, f32x4 hi) {
  bf16x8 r;
  r[0] = (__bf16)lo[0]; r[1] = (__bf16)lo[1]; r[2] = (__bf16)lo[2]; r[3] = (__bf16)lo[3];
  r[4] = (__bf16)hi[0]; r[5] = (__bf16)hi[1]; r[6] = (__bf16)hi[2]; r[7] = (__bf16)hi[3];
  return r;
}

__device__ __forceinline__ float wave_max_xor48(float x) {
  x = fmaxf(x, __shfl_xor(x, 16, 64));
  x = fmaxf(x, __shfl_xor(x, 32, 64));
  return x;
}
__device__ __forceinline__ float wave_sum_xor48(float x) {
  x += __shfl_xor(x, 16, 64);
  x += __shfl_xor(x, 32, 64);
  return x;
}


// ---- length-aware chunk plan ------------------------------------------------------------------
// With `items` = B * n_kv work items and G = n_wg > items workgroups, every workgroup derives the same
// plan from cur_pos: chunks are whole pairs of blocks (64 positions); row b has np_b pairs; the chunk
// length T (pairs) is the smallest of 64 candidates between ceil(W / G) and ceil(W / (G - items))
// (W = n_kv * sum_b np_b) for which n_kv * sum_b max(1, ceil(np_b / T)) <= G. The upper end always
// qualifies, since sum_b max(1, ceil(np_b / T)) <= W / (n_kv T) + B. Item (b, kvh) is cut into
// n_b = max(1, ceil(np_b / T)) near-equal chunks; chunks are numbered row by row, then KV head by KV
// head, and chunk number = workgroup index = workspace slot.

// n / d for 0 <= n < 2^22, 1 <= d, with 1/d precomputed: one float multiply, one correction step.
struct FDiv {
  int d;
  float r;
};
__device__ __forceinline__ FDiv make_fdiv(int d) { return FDiv{d, 1.0f / (float)d}; }
__device__ __forceinline__ int fdiv(int n, FDiv f) {
  int q = (int)((float)n * f.r);
  const int r = n - q * f.d;
  return q + (r >= f.d ? 1 : 0) - (r < 0 ? 1 : 0);
}
__device__ __forceinline__ int ceil_fdiv(int n, FDiv f) { return fdiv(n + f.d - 1, f); }

// A uniform int32 read through the scalar path (the data is not written during the kernel): it waits on
// the scalar counter, so vector loads issued around it are not held up by it.
__device__ __forceinline__ int load_uniform(const int32_t* p, long long i) {
  return reinterpret_cast<const __attribute__((address_space(4))) int32_t*>(reinterpret_cast<uintptr_t>(p))[i];
}

__device__ __forceinline__ int clamp_len(const DecodeArgs& a, int pos) {
  const int len = pos + 1;
  return len < 0 ? 0 : (len > a.S ? a.S : len);
}
__device__ __forceinline__ int row_len(const DecodeArgs& a, int b) { return clamp_len(a, load_uniform(a.cur_pos, b)); }

__device__ __forceinline__ int row_pairs(const DecodeArgs& a, int b) { return (row_len(a, b) + 63) >> 6; }

// The plan's chunk length T in pairs (the same value in every lane of every wave that calls it). The
// rows' positions are read through the scalar cache: one line holds 16 rows, so B rows cost a miss per
// 16 rows and hits for the rest.
__device__ int plan_chunk_pairs(const DecodeArgs& a) {
  const int lane = threadIdx.x & 63;
  const int G = a.n_wg, items = a.B * a.n_kv;
  int W = 0;
  for (int b = 0; b < a.B; ++b) W += row_pairs(a, b);
  W *= a.n_kv;
  const int lo = max(1, (W + G - 1) / G);
  const int hi = max(lo, (W + (G - items) - 1) / (G - items));
  const int step = max(1, (hi - lo + 62) / 63);
  const int T = lo + lane * step;           // lane 63: T >= hi
  const FDiv fT = make_fdiv(T);
  int C = 0;
  for (int b = 0; b < a.B; ++b) C += max(1, ceil_fdiv(row_pairs(a, b), fT));
  const unsigned long long ok = __ballot(C * a.n_kv <= G);
  return lo + __builtin_ctzll(ok) * step;
}

// LDS map of one workgroup (latent mode; full-K mode keeps only the merge buffer and the counter):
//   rtab  pair-relative K rotation (offset t < 64 inside a pair of blocks), fp16 x 4 {cos f, sin f,
//         cos f+1, sin f+1} per (block of the pair, tile, 16-dim row tile, lane); the packed fp16
//         multiplies take (cos, cos) and (-sin, sin) through operand selects and the negate modifier  16 KB
//   ukT   u_k^T, rows padded by 16 bytes (bank spread)                               HD x (RK + 8) bf16
//   qx    per wave, the rotated query (fp16) regrouped into its MFMA operand layout  NW x 4 KB
//   tl    (cos, sin) of angle 64*Lo*f, Lo < 16: the low part of a pair base           [16][64] float2
//   qs    the item's query rows (zero rows past rep), so the block loop issues no global load
//         besides the latent prefetch                                                 [16][128] bf16
//   ctr   the block counter
//   th    (cos, sin) of angle 1024*H*f, H < ceil(S / 1024): the high part             [nH][64] float2
//   kc    staging of cs_tab rows 0..7 and 8, 16, .., 56 ([row][f] float2) while rtab is built, overlaying qx
// The wave-merge buffer of the epilogue overlays the front.
template <int RK, int RV, bool KFULL, int NW, int IPW = 1>
struct Smem {
  static constexpr int UKT_STRIDE = RK + 8;
  static constexpr int RTAB_BYTES = KFULL ? 0 : 2 * 2 * 8 * 64 * 8;
  static constexpr int KC_BYTES = 15 * 64 * 8;   // the 15 staged cs_tab rows of the K rotation table
  static constexpr int UKT_BYTES = KFULL ? 0 : HD * UKT_STRIDE * 2;
  static constexpr int QX_WAVE_BYTES = 16 * 4 * 8 * 4 * 2;   // [head 16][g 4][row tile 8][4 dims] fp16
  static constexpr int QX_BYTES = KFULL ? 0 : (NW * QX_WAVE_BYTES > KC_BYTES ? NW * QX_WAVE_BYTES : KC_BYTES);
  static constexpr int TL_BYTES = KFULL ? 0 : 16 * 64 * 8;
  static constexpr int QS_BYTES = KFULL ? 0 : IPW * 16 * HD * 2;   // the query rows of each item
  static constexpr int UKT_OFFSET = RTAB_BYTES;
  static constexpr int QX_OFFSET = UKT_OFFSET + UKT_BYTES;
  static constexpr int TL_OFFSET = QX_OFFSET + QX_BYTES;
  static constexpr int QS_OFFSET = TL_OFFSET + TL_BYTES;
  static constexpr int MAIN_BYTES = QS_OFFSET + QS_BYTES;
  static constexpr int MERGE_BYTES = NW * 16 * (RV + 2) * 4;
  static constexpr int CTR_OFFSET = ((MAIN_BYTES > MERGE_BYTES ? MAIN_BYTES : MERGE_BYTES) + 15) & ~15;
  static constexpr int TH_OFFSET = CTR_OFFSET + 16;
  static_assert(KFULL || QX_BYTES >= KC_BYTES, "the cs_tab staging rows overlay qx");
  __host__ __device__ static int bytes(int S) { return TH_OFFSET + (KFULL ? 0 : ((S + 1023) / 1024) * 64 * 8); }
};

template <typename T>
__device__ __forceinline__ float4 load4f(const T* p);
template <>
__device__ __forceinline__ float4 load4f<float>(const float* p) { return *reinterpret_cast<const float4*>(p); }
template <>
__device__ __forceinline__ float4 load4f<__bf16>(const __bf16* p) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
}

// Last-finisher counting across the workgroups of one launch. Each of nc workgroups that produce parts
// of one result has written its part with system-scope stores (global stores that write through past
// the XCD's L2 to memory) and waited for them to complete; then one thread calls count_done, which adds
// the workgroup to the result's 8-byte counter with a system-scope compare-and-swap and returns true for
// the workgroup whose count completes the result. That workgroup reads the parts with system-scope loads
// (from memory, whichever XCD wrote them: no L2 write-back or invalidate, no fence) and leaves the
// counter at zero. A counter word carries a fixed tag and the call number in its upper 48 bits (tag,
// from next_epoch; its low 16 bits zero) and the count below; a word with other upper bits (another
// call's, memory never written) counts as zero, so counters need no clearing between calls.
__device__ __forceinline__ bool count_done(unsigned long long* ctr, unsigned long long tag, int nc) {
  unsigned long long old = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM), nw;
  int done;
  do {
    done = (((old & ~0xFFFFull) == tag) ? (int)(old & 0xFFFF) : 0) + 1;
    nw = tag | (unsigned long long)(done == nc ? 0 : done);
  } while (!__hip_atomic_compare_exchange_strong(ctr, &old, nw, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_SYSTEM));
  return done == nc;
}

// The workgroup-wide step before and around count_done: every thread's system-scope stores complete,
// thread 0 counts, and the answer (uniform) comes back through the LDS word *flag.
__device__ __forceinline__ bool workgroup_count_done(unsigned long long* ctr, unsigned long long tag, int nc, int* flag) {
  __builtin_amdgcn_s_waitcnt(0);            // this thread's part stores have completed
  __syncthreads();
  if (threadIdx.x == 0) flag[0] = count_done(ctr, tag, nc) ? 1 : 0;
  __syncthreads();
  return flag[0] != 0;
}

// A split item's chunks merge inside the decode launch (no second launch): each chunk's workgroup has
// written its partial (O, m, l) with system-scope stores, counts itself into the item's counter, and the
// workgroup that completes the item writes out = sum_s O_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), chunks in
// order: the result does not depend on which workgroup finishes last. smem: any LDS word no wave reads
// any more.
template <int RV, int NW, typename OutT>
__device__ __forceinline__ void merge_split_item(const DecodeArgs& a, char* smem, int first, int nc, int b, int kvh) {
  unsigned long long* ctr =
      reinterpret_cast<unsigned long long*>(a.ws + (long long)a.n_wg * 16 * (RV + 2)) + (b * a.n_kv + kvh);
  if (!workgroup_count_done(ctr, a.epoch, nc, reinterpret_cast<int*>(smem))) return;   // uniform
  constexpr int MC = 8;                     // chunk partials loaded together per round trip
  constexpr long long SLOT = 16 * (RV + 2);
  for (int e = threadIdx.x; e < a.rep * RV; e += NW * 64) {
    const int h = e / RV, r = e - h * RV;
    const float* ws = a.ws + ((long long)first * 16 + h) * (RV + 2);
    float M = NEG_INF, L = 0.f, acc = 0.f;
    for (int s0 = 0; s0 < nc; s0 += MC) {
      float mv[MC], lv[MC], ov[MC];
#pragma unroll
      for (int i = 0; i < MC; ++i) {
        const float* row = ws + min(s0 + i, nc - 1) * SLOT;   // clamped into the item's slots
        mv[i] = __hip_atomic_load(row + RV, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        lv[i] = __hip_atomic_load(row + RV + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        ov[i] = __hip_atomic_load(row + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
      float Mn = M;
#pragma unroll
      for (int i = 0; i < MC; ++i)
        if (s0 + i < nc) Mn = fmaxf(Mn, mv[i]);
      if (Mn == NEG_INF) continue;          // every chunk so far empty
      const float c = __builtin_amdgcn_exp2f(M - Mn);   // 0 while M is -inf
      L *= c;
      acc *= c;
#pragma unroll
      for (int i = 0; i < MC; ++i) {
        if (s0 + i < nc) {
          const float f = __builtin_amdgcn_exp2f(mv[i] - Mn);
          L += lv[i] * f;
          acc += ov[i] * f;
        }
      }
      M = Mn;
    }
    OutT* o = static_cast<OutT*>(a.out) + out_index(a, b, ((long long)kvh * a.rep + h) * RV + r, (long long)a.n_q * RV);
    store_out(o, L > 0.f ? acc / L : 0.f);
  }
}

// IPW items per workgroup: 2 runs two items of one KV head (batch rows b and b + B/2) on the two halves
// of the waves, which share the angle tables and u_k^T staged once.
template <int RK, int RV, bool KFULL, bool TILED, bool PAGED, int NW, typename TabT, typename OutT, int IPW = 1>
// 8 waves: two per SIMD, 256 registers each; 4 waves: one per SIMD with the whole register file.
__global__ __launch_bounds__(NW * 64, NW == 8 ? 2 : 1)
void palu_decode_kernel(const DecodeArgs a) {
  static_assert(RK % 16 == 0 && RK <= 128 && (TILED || RK % 32 == 0), "RK: 16-wide half tiles (tiled), 32-wide rows");
  static_assert(RV % 16 == 0 && RV <= 128 && (TILED || RV % 32 == 0), "RV: 16-wide V tiles (tiled), 32-wide rows");
  static_assert(!KFULL || RK == HD, "full K has the head dim");
  constexpr int KBF = RK / 32;              // 32-wide contraction blocks of the K operand
  constexpr bool KH = RK % 32 != 0;         // and a 16-wide one (tiled caches)
  constexpr int KB = KBF + (KH ? 1 : 0);    // register blocks; a half block holds 4 values, zeros above
  constexpr int VB = RV / 32;   // 32-wide blocks of a V row
  constexpr int VT = RV / 16;   // 16-wide V tiles = PV M-tiles
  using SM = Smem<RK, RV, KFULL, NW, IPW>;
  static_assert(IPW == 1 || (IPW == 2 && !PAGED && !KFULL), "two items per workgroup: contiguous latent caches");
  constexpr int NWI = NW / IPW;             // waves per item

  extern __shared__ __attribute__((aligned(16))) char smem[];
  f16x4* rtab = reinterpret_cast<f16x4*>(smem);
  __bf16* ukT = reinterpret_cast<__bf16*>(smem + SM::UKT_OFFSET);
  float2* tl = reinterpret_cast<float2*>(smem + SM::TL_OFFSET);
  float2* th = reinterpret_cast<float2*>(smem + SM::TH_OFFSET);
  float2* kc = reinterpret_cast<float2*>(smem + SM::QX_OFFSET);
  __bf16* qs_lds = reinterpret_cast<__bf16*>(smem + SM::QS_OFFSET);
  int* ctr = reinterpret_cast<int*>(smem + SM::CTR_OFFSET);
  int* pt_lds = reinterpret_cast<int*>(smem + SM::bytes(a.S));   // paged: this split's page ids

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index, held in a scalar register
  const int half = IPW == 1 ? 0 : w / NWI;                  // the wave's item slot
  const int wi = w - half * NWI;                            // wave index within its item
  const int n = lane & 15, g = lane >> 4;
  _Float16* qx = reinterpret_cast<_Float16*>(smem + SM::QX_OFFSET + w * SM::QX_WAVE_BYTES);

  // Latent mode: the angle-table rows are the same for every workgroup and depend on nothing below, so
  // their loads are issued first, ahead of the plan. Rows t < 64 serve the K rotation, 64*Lo (Lo < 16)
  // and 1024*H the query's pair base; one coalesced row per wave load.
  // Rows: t0 < 8 and 8 t1 (t1 = 1..7) for the K rotation (t = 8 t1 + t0 by angle addition), 64 Lo
  // (Lo < 16) and 1024 H (H < ceil(S / 1024)) for the query's pair base.
  const int n_rows = KFULL ? 0 : 31 + (a.S + 1023) / 1024;
  constexpr int RPW = (31 + 64 + NW - 1) / NW;  // rows per wave, enough for S <= 65536
  auto row_t = [](int r) { return r < 8 ? r : (r < 15 ? 8 * (r - 7) : (r < 31 ? 64 * (r - 15) : 1024 * (r - 31))); };
  float4 rowv[KFULL ? 1 : RPW];
  if constexpr (!KFULL) {
    const TabT* cs = static_cast<const TabT*>(a.cs);
    // Only the rows the sequence length needs are loaded (the branch is uniform): each row load is 16
    // cache lines for the CU's vector memory pipeline, and RPW rows per wave for every wave held the
    // second wave of each SIMD about 1.4 us behind the first before its loads went out.
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int r = w + i * NW;
      if (r < n_rows) {
        int t = row_t(r);
        t = t < a.cs_rows ? t : 0;
        rowv[i] = load4f(cs + (long long)t * (2 * HD) + 4 * lane);   // lane < 32: cos, else sin
      }
    }
  }

  // This workgroup's item and position range: the whole sequence of item blockIdx.x, or one chunk of
  // the length-aware plan (computed identically, and uniformly, by every wave).
  // A whole item's end (its row length) is read after the first latent blocks are issued, in the
  // prologue: those loads do not depend on it.
  int b, kvh, s_lo, s_hi = 0, n_chunks = 1, first_chunk = 0;
  if (!a.balanced) {
    const int item = blockIdx.x + half * a.n_wg;   // two items: n_wg = B * n_kv / 2, so the KV head is shared
    b = item / a.n_kv;
    kvh = item - b * a.n_kv;
    s_lo = 0;
  } else {
    const FDiv fT = make_fdiv(plan_chunk_pairs(a));
    int base = 0, rb = -1, np = 0;
    const int gid = blockIdx.x;
    for (int r = 0; r < a.B; ++r) {
      np = row_pairs(a, r);
      n_chunks = max(1, ceil_fdiv(np, fT));
      if (gid < base + a.n_kv * n_chunks) { rb = r; break; }
      base += a.n_kv * n_chunks;
    }
    if (rb < 0) return;                     // past the plan's last chunk (uniform: no barrier reached)
    const FDiv fn = make_fdiv(n_chunks);
    b = rb;
    kvh = fdiv(gid - base, fn);
    const int j = gid - base - kvh * n_chunks;
    first_chunk = gid - j;                  // the item's chunks are workgroups first_chunk .. + n_chunks - 1
    s_lo = 64 * fdiv(j * np, fn);
    s_hi = min(row_len(a, b), 64 * fdiv((j + 1) * np, fn));
  }
  b = __builtin_amdgcn_readfirstlane(b);
  kvh = __builtin_amdgcn_readfirstlane(kvh);
  s_lo = __builtin_amdgcn_readfirstlane(s_lo);
  n_chunks = __builtin_amdgcn_readfirstlane(n_chunks);
  first_chunk = __builtin_amdgcn_readfirstlane(first_chunk);
  const int grp = KFULL ? kvh : kvh / a.hpg;

  const __bf16* kbase = a.k + (PAGED ? 0 : b * a.k_sb) + grp * a.k_sg;
  const __bf16* vbase = a.v + (PAGED ? 0 : b * a.v_sb) + grp * a.v_sg;

  // Paged caches: page ids of the split's blocks, staged in LDS during the prologue (the first block
  // of each wave reads its id from global memory). Ids are clamped into the pool, so a bad page table
  // reads wrong rows but never leaves the allocation.
  const int pg_lo = PAGED ? ((s_lo >> 5) >> a.page_shift) : 0;
  const int bmask = PAGED ? (1 << a.page_shift) - 1 : 0;
  auto clamp_page = [&](int p) { return p < 0 ? 0 : (p >= a.n_pages ? a.n_pages - 1 : p); };
  auto page_global = [&](int base) -> int {
    if constexpr (!PAGED) return 0;
    return clamp_page(load_uniform(a.page_table, (long long)b * a.pt_stride + ((base >> 5) >> a.page_shift)));
  };
  auto page_lds = [&](int base) -> int {
    if constexpr (!PAGED) return 0;
    return clamp_page(__builtin_amdgcn_readfirstlane(pt_lds[((base >> 5) >> a.page_shift) - pg_lo]));
  };
  // Element offset of the 32-position block at position base (page pid when paged) in a stream of
  // width W whose page (or row) stride is page_stride.
  auto blk_off = [&](int base, int pid, long long page_stride, int W) -> long long {
    if constexpr (PAGED) return (long long)pid * page_stride + (long long)((base >> 5) & bmask) * (32 * W);
    return (long long)(base >> 5) * (32 * W);
  };

  // One block's K (latent or full) and V rows into registers.
  //   K, both layouts: register kd[c][kb] of lane (n, g) = width-index 32*kb + 8*g .. +7 of block
  //     position 8*(n/4) + 4*c + n%4 (the B operand of the rebuild, or the A operand of QK).
  //   V, TILED: register vd[mt] of lane (m = n, g) = block positions 8*g .. 8*g+7 of V column 16*mt + m,
  //     which is directly the A operand of O^T += V^T P^T.
  //   V, ROWS: register vd[c*VB + vb] holds the row pieces like K; an identity MFMA regroups them.
  // ROWS clamps rows past the cache end (their scores and values are masked). A load that is not live
  // (past the wave's last block) still issues the same instructions, at the block given, with every
  // lane on the block's first bytes (TILED), so the number of loads in flight is the same on every
  // path; its data is never used.
  auto row_in_blk = [&](int base, int c) {
    int t = 8 * (n >> 2) + 4 * c + (n & 3);     // position in the block
    if (!PAGED && base + t >= a.S) t = a.S - 1 - base;   // a page always holds whole blocks
    return t;
  };
  auto load_k = [&](int base, bool live, int pid, bf16x8 (&kd)[2][KB]) {
    if constexpr (TILED) {
      const __bf16* kt = kbase + blk_off(base, pid, a.k_sb, RK);
#pragma unroll
      for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb)
          kd[c][kb] = __builtin_nontemporal_load(
              reinterpret_cast<const bf16x8*>(kt + c * 16 * RK + kb * 512 + (live ? lane * 8 : 0)));
        if constexpr (KH)
          kd[c][KBF] = low4(__builtin_nontemporal_load(
              reinterpret_cast<const bf16x4*>(kt + c * 16 * RK + KBF * 512 + (live ? lane * 4 : 0))));
      }
    } else {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const __bf16* kr = kbase + blk_off(base, pid, a.k_sb, RK) + (long long)row_in_blk(base, c) * RK + 8 * g;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) kd[c][kb] = *reinterpret_cast<const bf16x8*>(kr + 32 * kb);
      }
    }
  };
  auto load_v = [&](int base, bool live, int pid, bf16x8 (&vd)[VT]) {
    if constexpr (TILED) {
      const __bf16* vt = vbase + blk_off(base, pid, a.v_sb, RV) + (live ? lane * 8 : 0);
#pragma unroll
      for (int mt = 0; mt < VT; ++mt)
        vd[mt] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(vt + mt * 512));
    } else {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const __bf16* vr = vbase + blk_off(base, pid, a.v_sb, RV) + (long long)row_in_blk(base, c) * RV + 8 * g;
#pragma unroll
        for (int vb = 0; vb < VB; ++vb) vd[c * VB + vb] = *reinterpret_cast<const bf16x8*>(vr + 32 * vb);
      }
    }
  };
  auto load_blk = [&](int base, bool live, int pid, bf16x8 (&kd)[2][KB], bf16x8 (&vd)[VT]) {
    load_k(base, live, pid, kd);
    load_v(base, live, pid, vd);
  };

  // Work is handed out in pairs of full blocks (pair p = blocks 2p, 2p + 1) from an LDS counter, so
  // that the waves of a workgroup finish together (which wave sums which blocks then depends on
  // timing, and each wave rounds its probabilities to bf16 against its own running max, so calls
  // differ at that rounding level); wave w starts on pair w. The deterministic schedule gives wave w
  // every NW-th pair. The loop runs complete pairs only; the one or two blocks left after them (an odd
  // full block, a partial last block) go to the wave whose next pair index is npairs, which exactly
  // one wave holds when the loop ends (the indices are w < NW, then counter values NW, NW + 1, ...).
  // (nfull and npairs follow the prologue, where a whole item's end is read.)
  if (tid < IPW) ctr[tid] = NWI;
  bf16x8 kl[2][KB], vl[VT], kln[2][KB], vln[VT];
  auto fence = []() __attribute__((always_inline)) { __builtin_amdgcn_sched_barrier(0); };
  // Block i (0, 1) of the wave's first pair, clamped inside the cache.
  auto load_first = [&](int i, bf16x8 (&kd)[2][KB], bf16x8 (&vd)[VT]) {
    const int f = min(s_lo + (2 * wi + i) * BLK, ((a.S - 1) / BLK) * BLK);
    const int pid = page_global(f);
    fence();
    load_blk(f, true, pid, kd, vd);
    fence();
  };

  // ---- prologue ----------------------------------------------------------------------------------
  // Latent mode: the angle tables and u_k^T go to LDS. The tables come from whole rows of cs_tab, one
  // coalesced row per wave load (rows t < 64 for K, 64*Lo and 1024*H for the query); these (L2) loads
  // are issued before the first latent block's (HBM) loads, so waiting on them does not wait on HBM.
  if constexpr (!KFULL) {
    // Every prologue load below is unconditional, its index clamped into the tensor: a load under a
    // branch makes the compiler wait for all outstanding loads where the branch joins, which would hold
    // the first latent block back until the tables had arrived.
    constexpr int UPT = (RK * (HD / 8) + NW * 64 - 1) / (NW * 64);
    bf16x8 ukv[UPT];
    const __bf16* ukp = a.w_rot + (long long)kvh * RK * (2 * HD);
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      int e = tid + i * NW * 64;         // consecutive lanes: consecutive ranks, one 8-column block
      e = e < RK * (HD / 8) ? e : 0;
      ukv[i] = *reinterpret_cast<const bf16x8*>(ukp + (long long)(e % RK) * (2 * HD) + (e / RK) * 8);
    }
    // query rows: 16 heads x 256 B, 16 bytes per thread for the first 256 threads of the item's waves
    // (zero rows past rep)
    const int qt = tid - half * NWI * 64;
    const int qh = qt >> 4, qc = (qt & 15) * 8;
    const bool qlive = qt < 16 * (HD / 8) && qh < a.rep;
    const bf16x8 qrow = *reinterpret_cast<const bf16x8*>(
        a.q + ((long long)b * a.n_q + (long long)kvh * a.rep + (qlive ? qh : 0)) * HD + (qlive ? qc : 0));
    // Every wave's table, u_k and query loads are issued before any wave's first latent block: the CU's
    // vector-memory pipeline serves them in order, so the (L2-hit) table loads of later waves do not
    // queue behind earlier waves' HBM latent loads.
    __syncthreads();
    // The wave's first block, issued before the row length is known (a wave whose first pair lies past
    // the row's data loads a block inside the cache instead and never uses it) and after every table
    // load: loads complete in issue order for the wait counter, so the prologue's waits on the tables
    // then leave this block in flight. The scheduling fences keep that order. The pair's second block
    // follows once the table registers are written out: issued with the first, it adds to the memory
    // traffic the staged loads queue behind (0.4-0.8 us per call slower at batch 32 x 8192 and 64 x 2048).
    load_first(0, kl, vl);
    if (!a.balanced) s_hi = row_len(a, b);
    if (qt < 16 * (HD / 8)) *reinterpret_cast<bf16x8*>(qs_lds + (half * 16 + qh) * HD + qc) = qlive ? qrow : bf16x8{};
    // rows -> [row][f] (cos, sin); lane l < 32 holds cos of f = 2l, 2l+1, lane l >= 32 the sines
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int r = w + i * NW;
      if (r < n_rows) {
        const int t = row_t(r);
        const bool ok = t < a.cs_rows;
        float2* dst = r < 15 ? kc + r * 64 : (r < 31 ? tl + (r - 15) * 64 : th + (r - 31) * 64);
        const int f = 2 * (lane & 31);
        float* d0 = reinterpret_cast<float*>(dst + f) + (lane >> 5);
        d0[0] = ok ? rowv[i].x : (lane < 32 ? 1.f : 0.f);
        d0[2] = ok ? rowv[i].z : (lane < 32 ? 1.f : 0.f);
      }
    }
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int e = tid + i * NW * 64;
      if (e < RK * (HD / 8)) {
        const int r = e % RK, d0 = (e / RK) * 8;
#pragma unroll
        for (int j = 0; j < 8; ++j) ukT[(d0 + j) * SM::UKT_STRIDE + r] = ukv[i][j];
      }
    }
    load_first(1, kln, vln);
    __syncthreads();
    // K rotation table in lane order: (cos, sin) of t f for t = 8 t1 + t0 < 64 by angle addition of the
    // staged rows t0 and 8 t1 in fp32 (within fp32 rounding of the table's own values, far below the
    // fp16 the table is stored in)
    for (int e = tid; e < 2 * 2 * 8 * 64; e += NW * 64) {
      const int l = e & 63, rt = (e >> 6) & 7, c = (e >> 9) & 1, hb = e >> 10;
      const int nn = l & 15, gg = l >> 4;
      const int t = 32 * hb + 8 * (nn >> 2) + 4 * c + (nn & 3);
      const int t0 = t & 7, t1 = t >> 3;
      const int f = 8 * rt + 2 * gg;
      float2 x = kc[t0 * 64 + f], y = kc[t0 * 64 + f + 1];       // (cos, sin) of t0 f and t0 (f + 1)
      if (t1 > 0) {
        const float2 u = kc[(7 + t1) * 64 + f], v = kc[(7 + t1) * 64 + f + 1];
        x = make_float2(x.x * u.x - x.y * u.y, x.y * u.x + x.x * u.y);
        y = make_float2(y.x * v.x - y.y * v.y, y.y * v.x + y.x * v.y);
      }
      rtab[e] = f16x4{(_Float16)x.x, (_Float16)x.y, (_Float16)y.x, (_Float16)y.y};
    }
  } else {
    load_first(0, kl, vl);
    load_first(1, kln, vln);
    if (!a.balanced) s_hi = row_len(a, b);
  }
  s_hi = __builtin_amdgcn_readfirstlane(s_hi);
  const int nblk = s_hi > s_lo ? (s_hi - s_lo + BLK - 1) / BLK : 0;
  const int nfull = s_hi > s_lo ? (s_hi - s_lo) / BLK : 0;   // an empty split (row shorter than s_lo) has none
  const int npairs = nfull >> 1;
  if constexpr (PAGED) {
    const int pg_hi = nblk > 0 ? (((s_hi - 1) >> 5) >> a.page_shift) : pg_lo - 1;
    for (int e = tid; e <= pg_hi - pg_lo; e += NW * 64)
      pt_lds[e] = clamp_page(a.page_table[(long long)b * a.pt_stride + pg_lo + e]);
  }
  __syncthreads();

  // Query rows of heads >= rep stay zero in the wave's regroup area, so every lane reads its operand.
  if constexpr (!KFULL) {
#pragma unroll
    for (int i = 0; i < SM::QX_WAVE_BYTES / (64 * 16); ++i)
      reinterpret_cast<float4*>(qx)[i * 64 + lane] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  // u_k^T as the A operand of the rebuild: row d = 16*rt + n, ranks 32*kb + 8*g + 0..7. Above
  // r_k = 64 it stays in LDS and is read per use.
  constexpr bool UK_LDS = !KFULL && RK > 64;
  bf16x8 ukA[UK_LDS ? 1 : 8][UK_LDS ? 1 : KB];
  if constexpr (!KFULL && !UK_LDS) {
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) {
#pragma unroll
      for (int kb = 0; kb < KBF; ++kb)
        ukA[rt][kb] = *reinterpret_cast<const bf16x8*>(ukT + (16 * rt + n) * SM::UKT_STRIDE + 32 * kb + 8 * g);
      if constexpr (KH)
        ukA[rt][KBF] = low4(*reinterpret_cast<const bf16x4*>(ukT + (16 * rt + n) * SM::UKT_STRIDE + 32 * KBF + 4 * g));
    }
  }

  // ROWS: identity B operands that move one 16-column slice of a 32-wide V block into the PV layout.
  bf16x8 idB[TILED ? 1 : 2];
  if constexpr (!TILED) {
#pragma unroll
    for (int par = 0; par < 2; ++par)
#pragma unroll
      for (int j = 0; j < 8; ++j) idB[par][j] = (8 * g + j == 16 * par + n) ? (__bf16)1.0f : (__bf16)0.0f;
  }

  f32x4 O[VT];
#pragma unroll
  for (int i = 0; i < VT; ++i) O[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = NEG_INF, l_run = 0.f;
  // The query operand: bf16 against full bf16 K; fp16 against the rebuilt K, which is rotated in fp16.
  using QV = typename std::conditional<KFULL, bf16x8, f16x8>::type;
  QV qB[4];

  // Query. Full-K mode: q * qscale once, head dim in natural order d = 32*kb + 8*g + j. Latent mode:
  // q~ = R_{-base} q * qscale per pair of blocks (base a multiple of 64). The rotation is spread over all 64 lanes (lane l owns query
  // head l/16 (+4, +8, +12 while < rep) and head dims 8*(l%16) .. +7, i.e. 4 frequency pairs), then
  // regrouped through the wave's LDS area into the operand order d(kb, g, j) =
  // 16*(2*kb + j/4) + 4*g + j%4 that the rebuilt K^T tile has in registers.
  const int qf = lane & 15;                 // dims 8*qf .. 8*qf + 7
  constexpr int QSLOTS = 4;                 // up to 16 query heads per KV head
  if constexpr (KFULL) {
    const bool qvalid = n < a.rep;
    const __bf16* qrow = a.q + ((long long)b * a.n_q + (long long)kvh * a.rep + (qvalid ? n : 0)) * HD;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const bf16x8 v = *reinterpret_cast<const bf16x8*>(qrow + 32 * kb + 8 * g);
#pragma unroll
      for (int j = 0; j < 8; ++j) qB[kb][j] = (__bf16)(qvalid ? (float)v[j] * a.qscale : 0.f);
    }
  }
  auto make_q = [&](int base) {
    // angle of the pair base 64*J, J = 16*H + Lo: (cos, sin) by angle addition of th[H] and tl[Lo]
    const int J = base >> 6;
    const float4* lo4 = reinterpret_cast<const float4*>(tl + (J & 15) * 64 + 4 * qf);
    const float4* hi4 = reinterpret_cast<const float4*>(th + (J >> 4) * 64 + 4 * qf);
    const float4 l01 = lo4[0], l23 = lo4[1], h01 = hi4[0], h23 = hi4[1];
    const float lc[4] = {l01.x, l01.z, l23.x, l23.z}, ls[4] = {l01.y, l01.w, l23.y, l23.w};
    const float hc[4] = {h01.x, h01.z, h23.x, h23.z}, hs[4] = {h01.y, h01.w, h23.y, h23.w};
    const float qsc = a.qscale;
    float cf[4], sf[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      cf[p] = (hc[p] * lc[p] - hs[p] * ls[p]) * qsc;
      sf[p] = (hs[p] * lc[p] + hc[p] * ls[p]) * qsc;
    }
    const int rt = qf >> 1, g0 = 2 * (qf & 1);
#pragma unroll
    for (int k = 0; k < QSLOTS; ++k) {
      const int h = g + 4 * k;
      if (h < a.rep) {
        const bf16x8 qv = *reinterpret_cast<const bf16x8*>(qs_lds + (half * 16 + h) * HD + 8 * qf);
        f16x4 y0, y1;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const float x0 = (float)qv[2 * p], x1 = (float)qv[2 * p + 1];
          const float r0 = x0 * cf[p] + x1 * sf[p], r1 = x1 * cf[p] - x0 * sf[p];  // R_{-base}
          if (p < 2) { y0[2 * p] = (_Float16)r0; y0[2 * p + 1] = (_Float16)r1; }
          else { y1[2 * p - 4] = (_Float16)r0; y1[2 * p - 3] = (_Float16)r1; }
        }
        // dims 16*rt + 4*g0 + 0..3 and 16*rt + 4*(g0+1) + 0..3 of head h
        *reinterpret_cast<f16x4*>(qx + ((h * 4 + g0) * 8 + rt) * 4) = y0;
        *reinterpret_cast<f16x4*>(qx + ((h * 4 + g0 + 1) * 8 + rt) * 4) = y1;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
      qB[kb] = __builtin_bit_cast(QV, *reinterpret_cast<const f16x8*>(qx + ((n * 4 + g) * 8 + 2 * kb) * 4));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  };

  // One block of 32 positions from the buffers (kc, vc). Only the last block of a range can be
  // partial; it runs the masked variant (PARTIAL), every other block carries no masking work.
  // after_k() runs once the K registers are consumed (scores done), before the softmax and PV: the
  // loop refills the K buffer there.
  auto compute = [&](auto partial_tag, int blk, const bf16x8 (&kc)[2][KB], const bf16x8 (&vc)[VT],
                     auto&& after_k) __attribute__((always_inline)) {
    constexpr bool PARTIAL = decltype(partial_tag)::value;
    const int base = s_lo + blk * BLK;
    const int hb = blk & 1;               // which block of its pair (s_lo is a multiple of 64)

    f32x4 sc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    if constexpr (KFULL) {
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) sc[c] = mfma16(kc[c][kb], qB[kb], sc[c]);
    } else {
      // One 32-dim slice of K^T (row tiles 2*kq, 2*kq + 1) at a time, for both position tiles:
      // rebuild, rotate, pack, and contract it with the matching query slice right away, so only
      // 16 accumulator registers are live instead of a whole 128 x 16 tile.
      // u_k^T rows from LDS (r_k > 64): the lane's row offset passes through an empty asm per block, so
      // the compiler re-reads the tiles where they are used instead of hoisting every tile of the
      // loop-invariant table into registers.
      int uk_off = n * SM::UKT_STRIDE + 8 * g;
      if constexpr (UK_LDS) asm volatile("" : "+v"(uk_off));
#pragma unroll
      for (int kq = 0; kq < 4; ++kq) {
        f32x4 acc[2][2];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int h = 0; h < 2; ++h) acc[c][h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < KBF; ++kb)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int rt = 2 * kq + h;
            bf16x8 ua;
            if constexpr (UK_LDS)
              ua = *reinterpret_cast<const bf16x8*>(ukT + uk_off + 16 * rt * SM::UKT_STRIDE + 32 * kb);
            else
              ua = ukA[rt][kb];
#pragma unroll
            for (int c = 0; c < 2; ++c) acc[c][h] = mfma16(ua, kc[c][kb], acc[c][h]);
          }
        if constexpr (KH) {
          // the last 16 ranks: lane (n, g) holds ranks 32 KBF + 4 g .. +3 of its u_k^T row and latent
          // column in the low half of both operands and zeros above, so the same 32-deep product (one
          // opcode on the whole accumulation chain) adds exactly their contribution
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int rt = 2 * kq + h;
            bf16x8 ua;
            if constexpr (UK_LDS)
              ua = low4(*reinterpret_cast<const bf16x4*>(ukT + uk_off - 4 * g + 16 * rt * SM::UKT_STRIDE + 32 * KBF));
            else
              ua = ukA[rt][KBF];
#pragma unroll
            for (int c = 0; c < 2; ++c) acc[c][h] = mfma16(ua, kc[c][KBF], acc[c][h]);
          }
        }
        // RoPE by the block offset of this lane's position, (x0, x1) -> (x0 c - x1 s, x1 c + x0 s), in
        // packed fp16: (x0, x1) * (c, c) + (x1, x0) * (-s, s) is one multiply and one fma per pair. The
        // rotated slice is the fp16 A operand of the QK product as it stands.
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          f16x2 r[2][2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            // (c, s) pairs: (c, c) and (-s, s) are the packed ops' operand selects and negate modifier
            const f16x4 t = rtab[((hb * 2 + c) * 8 + 2 * kq + h) * 64 + lane];
            const f16x2 c0 = {t[0], t[0]}, s0 = {-t[1], t[1]}, c1 = {t[2], t[2]}, s1 = {-t[3], t[3]};
            const f16x2 x01 = to_f16x2(acc[c][h][0], acc[c][h][1]);
            const f16x2 x23 = to_f16x2(acc[c][h][2], acc[c][h][3]);
            r[h][0] = x01 * c0 + x01.yx * s0;
            r[h][1] = x23 * c1 + x23.yx * s1;
          }
          const f16x8 kA = {r[0][0][0], r[0][0][1], r[0][1][0], r[0][1][1],
                            r[1][0][0], r[1][0][1], r[1][1][0], r[1][1][1]};
          sc[c] = mfma16(kA, qB[kq], sc[c]);
        }
      }
    }
    after_k();

    // Causal / range mask: score register i of tile c is position base + 8*g + 4*c + i.
    if constexpr (PARTIAL) {
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (base + 8 * g + 4 * c + i >= s_hi) sc[c][i] = NEG_INF;
    }

    // Online softmax, exp2 domain; lanes n, n+16, n+32, n+48 hold query head n. Each lane tests its
    // own scores against the running max; only when some score passes it by more than 2^8 does the
    // wave reduce the block max across lanes and refresh the running max.
    float bm = max8(sc[0], sc[1]);
    if (__any(bm > m_run + LAZY_RESCALE_LOG2)) {
      bm = wave_max_xor48(bm);
      const float mn = fmaxf(m_run, bm);
      const float alpha = (m_run == NEG_INF) ? 0.f : __builtin_amdgcn_exp2f(m_run - mn);
#pragma unroll
      for (int i = 0; i < VT; ++i) O[i] *= alpha;
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

    // O^T += V^T P^T. Masked positions are zeroed in V too (their cache rows may hold anything).
#pragma unroll
    for (int mt = 0; mt < VT; ++mt) {
      bf16x8 vA;
      if constexpr (TILED) {
        vA = vc[mt];
        if constexpr (PARTIAL) {
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (base + 8 * g + j >= s_hi) vA[j] = (__bf16)0.0f;
        }
      } else {
        f32x4 x0 = mfma16(vc[mt >> 1], idB[mt & 1], f32x4{0.f, 0.f, 0.f, 0.f});
        f32x4 x1 = mfma16(vc[VB + (mt >> 1)], idB[mt & 1], f32x4{0.f, 0.f, 0.f, 0.f});
        if constexpr (PARTIAL) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (base + 8 * g + i >= s_hi) x0[i] = 0.f;
            if (base + 8 * g + 4 + i >= s_hi) x1[i] = 0.f;
          }
        }
        vA = pack8(x0, x1);
      }
      O[mt] = mfma16(vA, pB, O[mt]);
    }
  };

  const std::integral_constant<bool, false> full_blk;
  const std::integral_constant<bool, true> partial_blk;
  // Pair loop. On entry the loads of pair p are issued: block 2p into (kl, vl), block 2p + 1 into
  // (kln, vln). Each buffer is refilled with the next pair's block as soon as its part is consumed: K
  // once the block's scores are done, V once its PV product is. Every load is issued unconditionally
  // (a dummy in-cache address when there is no next pair) and the loop body has no other branch, so
  // the compiler waits on exactly the loads a step consumes while about two blocks stream in.
  // The early K refill keeps one more K buffer live through the softmax and PV; it is used where
  // that still fits the register budget without spilling (full K, r_k <= 64, r_k + r_v <= 192; the
  // rest refill K together with V after the PV product).
  constexpr bool EARLY_K = KFULL || KB * 32 <= 64 || KB * 32 + RV <= 192;
  // The blocks left after the full pairs are loaded by the loop like a next pair (below) where both
  // stay in registers past the loop without spilling: every width but r_k <= 64 (u_k^T in registers)
  // with r_v >= 112 tiled or >= 96 row-major, whose waves take them one at a time after the loop.
  constexpr bool TAIL_REGS = KFULL || UK_LDS || RV + (TILED ? 0 : 16) < 112;
  int p = wi;
  while (p < npairs) {
    int pn = p + NWI;
    if (!a.deterministic) {
      // readfirstlane keeps the pair index in a scalar register: the loop branches stay uniform.
      int got = 0;
      if (lane == 0) got = atomicAdd(ctr + half, 1);
      pn = __builtin_amdgcn_readfirstlane(got);
    }
    const int b0 = 2 * p;
    const bool hasn = pn < npairs;
    // Index npairs stands for the blocks left after the full pairs (an odd full block and / or the
    // partial last block): the wave that draws it loads them like a pair here, so they are in its
    // registers when the loop ends instead of loaded one at a time after it. A missing second one reads
    // the current pair's second block (in the cache; never used).
    const bool tailn = TAIL_REGS && pn == npairs && 2 * npairs < nblk;
    const bool ln0 = hasn || tailn, ln1 = hasn || (tailn && 2 * npairs + 1 < nblk);
    const int nb0 = s_lo + (ln0 ? 2 * pn : b0) * BLK, nb1 = ln1 ? nb0 + BLK : s_lo + (b0 + 1) * BLK;
    const int pid0 = page_lds(nb0), pid1 = page_lds(nb1);
    if constexpr (!KFULL) make_q(s_lo + b0 * BLK);   // one query rotation serves both blocks of the pair
    compute(full_blk, b0, kl, vl, [&] {
      if constexpr (EARLY_K) { fence(); load_k(nb0, ln0, pid0, kl); fence(); }
    });
    fence();
    if constexpr (!EARLY_K) load_k(nb0, ln0, pid0, kl);
    load_v(nb0, ln0, pid0, vl);
    fence();
    compute(full_blk, b0 + 1, kln, vln, [&] {
      if constexpr (EARLY_K) { fence(); load_k(nb1, ln1, pid1, kln); fence(); }
    });
    fence();
    if constexpr (!EARLY_K) load_k(nb1, ln1, pid1, kln);
    load_v(nb1, ln1, pid1, vln);
    fence();
    p = pn;
  }
  if (p == npairs && 2 * npairs < nblk) {
    auto none = [] {};
    const int e0 = 2 * npairs;
    if constexpr (!KFULL) make_q(s_lo + e0 * BLK);
    if constexpr (TAIL_REGS) {
      // The blocks left after the full pairs, already in (kl, vl) and (kln, vln): loaded in this wave's
      // last loop step, or as its first pair in the prologue when it drew no full pair. The second,
      // when there is one, is the partial last block.
      if (e0 < nfull) compute(full_blk, e0, kl, vl, none);
      else compute(partial_blk, e0, kl, vl, none);
      if (e0 + 1 < nblk) compute(partial_blk, e0 + 1, kln, vln, none);
    } else {
      // one at a time (both held in registers would not fit this width's register budget)
      for (int e = e0; e < nblk; ++e) {
        const int base = s_lo + e * BLK;
        load_blk(base, true, page_lds(base), kl, vl);
        if (e < nfull) compute(full_blk, e, kl, vl, none);
        else compute(partial_blk, e, kl, vl, none);
      }
    }
  }

  // ---- merge the NW wave partials of this workgroup ---------------------------------------------
  l_run = wave_sum_xor48(l_run);
  __syncthreads();  // the merge buffer overlays the tables
  float* mbuf = reinterpret_cast<float*>(smem);
  if (n < a.rep) {
    float* row = mbuf + (w * 16 + n) * (RV + 2);
    if (g == 0) { row[RV] = m_run; row[RV + 1] = l_run; }
#pragma unroll
    for (int mt = 0; mt < VT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) row[16 * mt + 4 * g + i] = O[mt][i];
  }
  __syncthreads();
  for (int e = tid; e < IPW * a.rep * RV; e += NW * 64) {
    const int slot = IPW == 1 ? 0 : e / (a.rep * RV);     // the item whose waves' partials this merges
    const int e2 = e - slot * a.rep * RV;
    const int h = e2 / RV, r = e2 - h * RV;
    float M = NEG_INF;
#pragma unroll
    for (int ww = 0; ww < NWI; ++ww) M = fmaxf(M, mbuf[((slot * NWI + ww) * 16 + h) * (RV + 2) + RV]);
    float L = 0.f, acc = 0.f;
    if (M != NEG_INF) {
#pragma unroll
      for (int ww = 0; ww < NWI; ++ww) {
        const float* row = mbuf + ((slot * NWI + ww) * 16 + h) * (RV + 2);
        const float f = __builtin_amdgcn_exp2f(row[RV] - M);
        L += row[RV + 1] * f;
        acc += row[r] * f;
      }
    }
    if (n_chunks == 1) {
      const int bs = IPW == 1 ? b : (blockIdx.x + slot * a.n_wg) / a.n_kv;
      OutT* o = static_cast<OutT*>(a.out) + out_index(a, bs, ((long long)kvh * a.rep + h) * RV + r, (long long)a.n_q * RV);
      store_out(o, L > 0.f ? acc / L : 0.f);
    } else {
      // the chunk's partial, written through to memory (system-scope stores bypass the XCD's L2, so the
      // workgroup that merges it reads it from any XCD without a cache write-back)
      float* wrow = a.ws + ((long long)blockIdx.x * 16 + h) * (RV + 2);
      __hip_atomic_store(wrow + r, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      if (r == 0) {
        __hip_atomic_store(wrow + RV, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(wrow + RV + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
    }
  }
  if (n_chunks > 1) merge_split_item<RV, NW, OutT>(a, smem, first_chunk, n_chunks, b, kvh);
}

template <int RK, int RV, bool KFULL, bool TILED, bool PAGED, typename TabT, typename OutT, int NW, int IPW = 1>
int launch_nw(const DecodeArgs& a, hipStream_t stream) {
  using SM = Smem<RK, RV, KFULL, NW, IPW>;
  auto kern = palu_decode_kernel<RK, RV, KFULL, TILED, PAGED, NW, TabT, OutT, IPW>;
  const int lds = SM::bytes(a.S) + (PAGED ? ((a.S >> 5 >> a.page_shift) + 2) * 4 : 0);
  if (lds > 160 * 1024) return fail(PALU_EUNSUPPORTED, "seq_len %d needs %d bytes of LDS (max 163840)", a.S, lds);
  static int attr_set = 0;
  if (attr_set < lds) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return fail(PALU_EHIP, "hipFuncSetAttribute: %s", hipGetErrorString(e));
    attr_set = lds;
  }
  hipLaunchKernelGGL(kern, dim3(a.n_wg), dim3(NW * 64), lds, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PALU_EHIP, "decode kernel launch: %s", hipGetErrorString(e));
  return PALU_OK;
}

template <int RK, int RV, bool KFULL, bool TILED, bool PAGED, typename TabT, typename OutT>
int launch(const DecodeArgs& a0, hipStream_t stream) {
  constexpr int NW = pick_nw<RK, RV, KFULL, TILED>();
  DecodeArgs a = a0;
  const int items = a.B * a.n_kv;
  a.n_wg = decode_workgroups(items);
  a.balanced = a.n_wg > items ? 1 : 0;
  if (!a.balanced) a.n_wg = items;
  // Chunks of the length-aware plan are short: there the fixed block order (no round trip to the
  // shared counter per pair) is the faster one, and it is reproducible as well.
  if (a.balanced) a.deterministic = 1;
  a.epoch = a.balanced ? next_epoch() : 0;
  const size_t need = decode_ws_bytes(items, RV);
  if (need > 0 && (a.ws == nullptr || a.ws_bytes < need))
    return fail(PALU_EINVAL, "workspace of %zu bytes needed (palu_decode_workspace_bytes), got %zu", need, a.ws_bytes);
  // Two or more whole items per CU (e.g. batch 64 x 8 KV heads): an 8-wave workgroup fills a CU's
  // registers, so the CU's second item would start, prologue and all, only when its first ended. One
  // 8-wave workgroup runs two items of one KV head instead (rows b and b + B/2, four waves each), so the
  // CU streams both at once and stages the angle tables and u_k^T once for the two. Built for the
  // tiled contiguous caches with fp32 tables and bf16 output, the decoder's configuration.
  if constexpr (NW == 8 && TILED && !PAGED && !KFULL && std::is_same<TabT, float>::value &&
                std::is_same<OutT, __bf16>::value) {
    if (!a.balanced && items >= 2 * TARGET_WGS && a.B % 2 == 0 &&
        Smem<RK, RV, KFULL, 8, 2>::bytes(a.S) <= 160 * 1024) {
      a.n_wg = items / 2;
      return launch_nw<RK, RV, KFULL, TILED, PAGED, TabT, OutT, 8, 2>(a, stream);
    }
  }
  return launch_nw<RK, RV, KFULL, TILED, PAGED, TabT, OutT, NW>(a, stream);
}

template <int RK, bool KFULL, bool TILED, bool PAGED, typename TabT, typename OutT>
int dispatch_rv(const DecodeArgs& a, int rv, hipStream_t s) {
  switch (rv) {
    case 32: return launch<RK, 32, KFULL, TILED, PAGED, TabT, OutT>(a, s);
    case 64: return launch<RK, 64, KFULL, TILED, PAGED, TabT, OutT>(a, s);
    case 96: return launch<RK, 96, KFULL, TILED, PAGED, TabT, OutT>(a, s);
    case 128: return launch<RK, 128, KFULL, TILED, PAGED, TabT, OutT>(a, s);
  }
  // V tiles are 16 wide, so tiled V caches also take the widths in between (row-major ones do not)
  if constexpr (TILED) {
    switch (rv) {
      case 48: return launch<RK, 48, KFULL, TILED, PAGED, TabT, OutT>(a, s);
      case 80: return launch<RK, 80, KFULL, TILED, PAGED, TabT, OutT>(a, s);
      case 112: return launch<RK, 112, KFULL, TILED, PAGED, TabT, OutT>(a, s);
    }
  }
  return fail(PALU_EUNSUPPORTED, "head_dim_v %d: this build supports V widths 32, 64, 96, 128 (and 48, 80, 112 for "
                                 "tiled caches)", rv);
}

// K16: the widths that end in a half tile (tiled caches only), built in translation units of their own.
template <bool TILED, bool PAGED, bool K16, typename TabT, typename OutT>
int dispatch_latent(const DecodeArgs& a, int rk, int rv, hipStream_t s) {
  if constexpr (K16) {
    static_assert(TILED, "half K tiles exist in the tiled layout only");
    switch (rk) {
      case 48: return dispatch_rv<48, false, TILED, PAGED, TabT, OutT>(a, rv, s);
      case 80: return dispatch_rv<80, false, TILED, PAGED, TabT, OutT>(a, rv, s);
      case 112: return dispatch_rv<112, false, TILED, PAGED, TabT, OutT>(a, rv, s);
    }
  } else {
    switch (rk) {
      case 32: return dispatch_rv<32, false, TILED, PAGED, TabT, OutT>(a, rv, s);
      case 64: return dispatch_rv<64, false, TILED, PAGED, TabT, OutT>(a, rv, s);
      case 96: return dispatch_rv<96, false, TILED, PAGED, TabT, OutT>(a, rv, s);
      case 128: return dispatch_rv<128, false, TILED, PAGED, TabT, OutT>(a, rv, s);
    }
  }
  return fail(PALU_EUNSUPPORTED, "r_k %d: this build rebuilds K from latents of width 32, 64, 96 or 128 (and 48, 80, "
                                 "112 for tiled caches)", rk);
}


// The four (table dtype, output dtype) instantiations of one cache layout.
template <bool TILED, bool PAGED, bool K16 = false>
int dispatch_dtypes(const DecodeArgs& a, int rk, int rv, int cs_dtype, int out_dtype, hipStream_t s) {
  const bool f32o = out_dtype == PALU_DTYPE_F32;
  if (cs_dtype == PALU_DTYPE_F32)
    return f32o ? dispatch_latent<TILED, PAGED, K16, float, float>(a, rk, rv, s)
                : dispatch_latent<TILED, PAGED, K16, float, __bf16>(a, rk, rv, s);
  return f32o ? dispatch_latent<TILED, PAGED, K16, __bf16, float>(a, rk, rv, s)
              : dispatch_latent<TILED, PAGED, K16, __bf16, __bf16>(a, rk, rv, s);
}

}  // namespace
