// C-ABI of libpalu_mi355x.so (declarations and argument meaning: include/palu_mi355x.h): argument
// validation with the reference op's messages, the latent-append kernel, and dispatch to the decode
// translation units.
#include "palu_kernel.h"

#include <atomic>
#include <mutex>

namespace palu {

thread_local char g_err[1024] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

unsigned long long next_epoch() {
  static std::atomic<unsigned long long> calls{0};
  return CHUNK_TAG | (((calls.fetch_add(1) + 1) & 0xFFFFFFFFull) << 16);
}

}  // namespace palu

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_layout(int layout, int seq_len, const char* who) {
  if (layout != PALU_LAYOUT_ROWS && layout != PALU_LAYOUT_TILED)
    return fail(PALU_EINVAL, "%s: cache layout must be PALU_LAYOUT_ROWS or PALU_LAYOUT_TILED, got %d", who, layout);
  if (layout == PALU_LAYOUT_TILED && seq_len % 32 != 0)
    return fail(PALU_EINVAL, "%s: a tiled cache holds whole 32-position blocks; seq_len %d is not a multiple of 32", who,
                seq_len);
  return PALU_OK;
}

// Paged pools: page_size a power of two in 32..4096 (whole 32-position blocks per page), at least one
// page, a page table of max_pages_per_seq entries per row. Returns log2(page_size / 32) in *shift.
int check_pages(const int32_t* page_table, int num_pages, int page_size, int max_pages, int* shift, const char* who) {
  if (!page_table) return fail(PALU_EINVAL, "%s: page_table is null", who);
  if (page_size < 32 || page_size > 4096 || (page_size & (page_size - 1)) != 0)
    return fail(PALU_EINVAL, "%s: page_size must be a power of two in 32..4096, got %d", who, page_size);
  if (num_pages <= 0 || max_pages <= 0)
    return fail(PALU_EINVAL, "%s: num_pages and max_pages_per_seq must be positive, got %d and %d", who, num_pages,
                max_pages);
  if ((long long)max_pages * page_size > 65536)
    return fail(PALU_EUNSUPPORTED, "%s: max_pages_per_seq * page_size = %lld positions; this build covers 65536", who,
                (long long)max_pages * page_size);
  int s = 0;
  while ((32 << s) < page_size) ++s;
  *shift = s;
  return PALU_OK;
}

// Latent append: cache[b, g, idx[b], :] = rows[b * sb + g * sg + 0 .. width - 1]; each thread moves 8
// consecutive values. A
// contiguous cache is [B, G, S, width]; a paged pool is [n_pages, G, S, width] with S the page size,
// and position p of row b lives on page page_table[b * pt_stride + p / S] (ids outside the pool skip
// the row).
template <int LAYOUT, bool PAGED>
__global__ __launch_bounds__(256) void palu_append_kernel(__bf16* cache, const __bf16* rows, long long sb,
                                                          long long sg, const int32_t* idx,
                                                          const int32_t* page_table, int pt_stride, int n_pages,
                                                          int B, int G, int S, int width) {
  const int vec = width / 8;
  const long long total = (long long)B * G * vec;
  for (long long e = blockIdx.x * (long long)blockDim.x + threadIdx.x; e < total; e += (long long)gridDim.x * blockDim.x) {
    const int v = (int)(e % vec);
    const long long bg = e / vec;
    const int b = (int)(bg / G), gi = (int)(bg - (long long)b * G);
    int p = idx[b];
    long long slab;
    if constexpr (PAGED) {
      if (p < 0 || p >= pt_stride * S) continue;
      const int pid = page_table[(long long)b * pt_stride + p / S];
      if (pid < 0 || pid >= n_pages) continue;
      slab = (long long)pid * G + gi;
      p &= S - 1;
    } else {
      if (p < 0 || p >= S) continue;
      slab = bg;
    }
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(rows + b * sb + gi * sg + 8 * v);
    __bf16* stream = cache + slab * S * width;
    if constexpr (LAYOUT == PALU_LAYOUT_ROWS) {
      *reinterpret_cast<bf16x8*>(stream + (long long)p * width + 8 * v) = x;
    } else if constexpr (LAYOUT == PALU_LAYOUT_TILED) {
      store_k8(stream, p, 8 * v, width, x);
    } else {
      const long long o = tiled_v_offset(p, 8 * v, width);   // 8 slots 16 bytes apart
#pragma unroll
      for (int j = 0; j < 8; ++j) stream[o + 8 * j] = x[j];
    }
  }
}

template <bool PAGED>
int launch_append(void* cache, const void* new_rows, const int32_t* update_idxs, const int32_t* page_table,
                  int pt_stride, int n_pages, int batch, int n_groups, int S, int width, int layout, hipStream_t stream,
                  long long sb = -1, long long sg = -1) {
  if (sb < 0) { sb = (long long)n_groups * width; sg = width; }
  const long long total = (long long)batch * n_groups * (width / 8);
  int blocks = (int)((total + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  auto* c = static_cast<__bf16*>(cache);
  auto* r = static_cast<const __bf16*>(new_rows);
  if (layout == PALU_LAYOUT_TILED)
    hipLaunchKernelGGL((palu_append_kernel<PALU_LAYOUT_TILED, PAGED>), dim3(blocks), dim3(256), 0, stream, c, r, sb, sg,
                       update_idxs, page_table, pt_stride, n_pages, batch, n_groups, S, width);
  else if (layout == PALU_LAYOUT_TILED_V)
    hipLaunchKernelGGL((palu_append_kernel<PALU_LAYOUT_TILED_V, PAGED>), dim3(blocks), dim3(256), 0, stream, c, r, sb, sg,
                       update_idxs, page_table, pt_stride, n_pages, batch, n_groups, S, width);
  else
    hipLaunchKernelGGL((palu_append_kernel<PALU_LAYOUT_ROWS, PAGED>), dim3(blocks), dim3(256), 0, stream, c, r, sb, sg,
                       update_idxs, page_table, pt_stride, n_pages, batch, n_groups, S, width);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PALU_EHIP, "append kernel launch: %s", hipGetErrorString(e));
  return PALU_OK;
}

// Append into grouped latents stored compactly (PALU_LAYOUT_TILED_GROUPED): row b's group streams lie one
// after another, group g at element offset off[g] of the row (row_elems elements per row) and width[g]
// wide; the source holds group g's row at rows + b * sb + g * sg (its first width[g] values). One
// thread per 8 values; vec0 are the groups' first vector indices within a row.
struct GroupTable {
  long long off[MAX_GROUPS];
  int width[MAX_GROUPS];
  int vec0[MAX_GROUPS + 1];
};

template <int LAYOUT>
__global__ __launch_bounds__(256) void palu_append_grouped_kernel(__bf16* cache, const __bf16* rows, long long sb,
                                                                  long long sg, const int32_t* idx, int B, int G, int S,
                                                                  long long row_elems, const GroupTable t) {
  const int vec = t.vec0[G];
  const long long total = (long long)B * vec;
  for (long long e = blockIdx.x * 256LL + threadIdx.x; e < total; e += (long long)gridDim.x * 256) {
    const int b = (int)(e / vec), u = (int)(e - (long long)b * vec);
    int gi = 0;
    while (gi + 1 < G && u >= t.vec0[gi + 1]) ++gi;
    const int v = u - t.vec0[gi];
    const int p = idx[b];
    if (p < 0 || p >= S) continue;
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(rows + b * sb + gi * sg + 8 * v);
    __bf16* stream = cache + b * row_elems + t.off[gi];
    if constexpr (LAYOUT == PALU_LAYOUT_TILED) {
      store_k8(stream, p, 8 * v, t.width[gi], x);
    } else {
      const long long o = tiled_v_offset(p, 8 * v, t.width[gi]);   // 8 slots 16 bytes apart
#pragma unroll
      for (int j = 0; j < 8; ++j) stream[o + 8 * j] = x[j];
    }
  }
}

int check_append(void* cache, const void* new_rows, const int32_t* update_idxs, int batch, int n_groups, int S,
                 int width, int layout, const char* who) {
  if (!cache || !new_rows || !update_idxs) return fail(PALU_EINVAL, "%s: a required pointer is null", who);
  if (batch <= 0 || n_groups <= 0 || S <= 0 || width <= 0 || width % 8 != 0)
    return fail(PALU_EINVAL, "%s: width must be a positive multiple of 8, got %d", who, width);
  if (int rc = check_layout(layout == PALU_LAYOUT_TILED_V ? PALU_LAYOUT_TILED : layout, S, who)) return rc;
  if (layout == PALU_LAYOUT_TILED && width % 16 != 0)
    return fail(PALU_EINVAL, "%s: a tiled K cache row is a multiple of 16 wide, got %d", who, width);
  if (layout == PALU_LAYOUT_TILED_V && width % 16 != 0)
    return fail(PALU_EINVAL, "%s: a tiled V cache row is a multiple of 16 wide, got %d", who, width);
  if (!aligned16(cache) || !aligned16(new_rows)) return fail(PALU_EINVAL, "%s: 16-byte alignment required", who);
  return PALU_OK;
}

// Fused epilogue of the decode step's QKV projection (its fp32 k-slice partials [ks][B][ncols]): per
// batch row, the q heads rotated at pos[b] into q_out and each latent group's K and V slices appended to
// the caches at pos[b] (QkvEpi), as palu_rope_rows and palu_latent_append_strided do over a bf16
// projection output. One thread per 8 consecutive columns; the partials are summed in slice order in
// fp32 and rounded once.
constexpr int QP_PK = 4;   // partial slices loaded together

__global__ __launch_bounds__(256) void palu_qkv_post_kernel(const float* part, int ks, int B, int ncols, QkvEpi e) {
  const int qv = e.nh * (HD / 8), kv = e.G * (e.k_w / 8), vv = e.G * (e.v_w / 8);
  const int per = qv + kv + vv;
  const long long total = (long long)B * per;
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
    const int b = (int)(i / per), t = (int)(i - (long long)b * per);
    int kind, gi, c8, col;
    if (t < qv) {
      kind = 0;
      c8 = (t % (HD / 8)) * 8;
      gi = t / (HD / 8);
      col = gi * HD + c8;
    } else if (t < qv + kv) {
      kind = 1;
      gi = (t - qv) / (e.k_w / 8);
      c8 = ((t - qv) % (e.k_w / 8)) * 8;
      col = e.k_off + gi * e.k_gs + c8;
    } else {
      kind = 2;
      gi = (t - qv - kv) / (e.v_w / 8);
      c8 = ((t - qv - kv) % (e.v_w / 8)) * 8;
      col = e.v_off + gi * e.v_gs + c8;
    }
    // The row's position and the first QP_PK partial slices are loaded together (the kernel is bound by
    // memory latency); slices past ks re-read the last one and are not added.
    const int p = e.pos[b];
    const float* pp = part + (long long)b * ncols + col;
    const long long pstride = (long long)B * ncols;
    f32x4 pa[QP_PK][2];
#pragma unroll
    for (int k = 0; k < QP_PK; ++k) {
      const float* pk = pp + min(k, ks - 1) * pstride;
      pa[k][0] = *reinterpret_cast<const f32x4*>(pk);
      pa[k][1] = *reinterpret_cast<const f32x4*>(pk + 4);
    }
    f32x4 s0 = pa[0][0], s1 = pa[0][1];
#pragma unroll
    for (int k = 1; k < QP_PK; ++k) {
      if (k < ks) {
        s0 += pa[k][0];
        s1 += pa[k][1];
      }
    }
    for (int k = QP_PK; k < ks; ++k) {
      s0 += *reinterpret_cast<const f32x4*>(pp + k * pstride);
      s1 += *reinterpret_cast<const f32x4*>(pp + k * pstride + 4);
    }
    float v[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
    qkv_store<8>(e, b, p, kind, gi, c8, v);
  }
}

int sdpa_setup(DecodeArgs& a, const void* q, const void* k_latent, const void* w_rot, const void* cs_tab,
               const void* v_latent, int head_dim_v, const int32_t* cur_pos, void* out, const float* rot_step,
               const void* trans_mat, const void* u_v, const int32_t* group_ranks, float scale, int heads_per_core,
               int rot_mode, int k_chunk,
               int batch, int n_q, int n_kv, int n_groups, int seq_len, int r_k, int r_v, int w_rot_width, int cs_rows,
               int cs_cols, int cs_dtype, int& out_dtype, int cache_layout, int deterministic, void* workspace,
               size_t workspace_bytes, const char* who) {
  if (!q || !k_latent || !w_rot || !cs_tab || !v_latent || !cur_pos || !out)
    return fail(PALU_EINVAL, "%s: a required tensor pointer is null", who);
  int grouped_streams = 0;
  if (rot_mode < 0 || rot_mode > 2) return fail(PALU_EINVAL, "rot_mode must be 'legacy', 'pack' or 'dst'");
  if ((rot_step == nullptr) != (trans_mat == nullptr))
    return fail(PALU_EINVAL, "rot_step and trans_mat are optional together: pass both (Phase 2) or neither (Phase 1)");
  if (rot_step == nullptr && k_chunk > 128)
    return fail(PALU_EINVAL, "Phase 1 streams the angle table per chunk and needs k_chunk_size <= 128, got %d", k_chunk);
  if (k_chunk < 0 || (k_chunk > 0 && (k_chunk % 32 != 0 || (k_chunk & (k_chunk - 1)) != 0)))
    return fail(PALU_EINVAL, "k_chunk_size must be 0 or a power of two multiple of 32, got %d", k_chunk);
  if (batch <= 0 || n_q <= 0 || n_kv <= 0 || n_groups <= 0 || seq_len <= 0)
    return fail(PALU_EINVAL, "%s: batch, head counts and seq_len must be positive", who);
  // Per-head (absorbed-V) tiled caches take latent widths in multiples of 16: V tiles are 16 wide and a K
  // row's last 16 columns form a half tile. Row-major caches and grouped latents (u_v) keep multiples of 32.
  const int r_step = (cache_layout == PALU_LAYOUT_TILED && u_v == nullptr) ? 16 : 32;
  if (r_k <= 0 || r_k % r_step != 0 || r_k > 512)
    return fail(PALU_EINVAL, "r_k must be a multiple of %d in %d..512 (the latent width of k_latent), got %d", r_step,
                r_step, r_k);
  const int rv_step = r_step;
  if (r_v <= 0 || r_v % rv_step != 0 || r_v > 512)
    return fail(PALU_EINVAL, "r_v must be a multiple of %d in %d..512 (the latent width of v_latent), got %d", rv_step,
                rv_step, r_v);
  if (n_kv % n_groups != 0)
    return fail(PALU_EINVAL, "heads_per_group: %d latent heads do not divide the %d KV heads of w_rot", n_groups, n_kv);
  const int hpg = n_kv / n_groups;
  if (w_rot_width != 2 * HD)
    return fail(PALU_EINVAL, "w_rot must be [1, n_kv, r_k, %d] = [u_k | u_k T], got last dim %d", 2 * HD, w_rot_width);
  if (cs_cols != 2 * HD) return fail(PALU_EINVAL, "cs_tab must be [1, 1, S, %d] = [cos | sin], got last dim %d", 2 * HD, cs_cols);
  if (cs_rows < seq_len)
    return fail(PALU_EINVAL, "cs_tab has %d rows but the latent cache has %d positions", cs_rows, seq_len);
  if (seq_len > 65536)
    return fail(PALU_EUNSUPPORTED, "seq_len %d: this build's block-angle tables cover 65536 positions", seq_len);
  if (n_q % n_kv != 0 || n_q / n_kv > 16)
    return fail(PALU_EINVAL, "KV head count %d must divide the %d query heads with at most 16 query heads per KV head", n_kv, n_q);
  if (heads_per_core > 1) {
    if (heads_per_core > n_kv)
      return fail(PALU_EINVAL, "heads_per_core %d exceeds the KV head count %d", heads_per_core, n_kv);
    if (hpg == 1) return fail(PALU_EINVAL, "heads_per_core > 1 shares a latent between heads and needs grouped latents");
    if (hpg % heads_per_core != 0)
      return fail(PALU_EINVAL, "heads_per_core %d must divide heads_per_group %d", heads_per_core, hpg);
  }
  if (cache_layout == PALU_LAYOUT_TILED_GROUPED) {
    if (u_v == nullptr || group_ranks == nullptr)
      return fail(PALU_EINVAL, "PALU_LAYOUT_TILED_GROUPED stores grouped latents at the groups' own ranks: it needs "
                               "u_v and group_ranks");
    cache_layout = PALU_LAYOUT_TILED;   // same tile orders, per-group streams (set at dispatch)
    grouped_streams = 1;
  }
  if (u_v != nullptr) {
    if (head_dim_v != HD) return fail(PALU_EINVAL, "head_dim_v must be %d when u_v rebuilds V in-kernel, got %d", HD, head_dim_v);
    if (n_groups > MAX_GROUPS)
      return fail(PALU_EUNSUPPORTED, "u_v: %d latent groups (the grouped-latent kernels take up to %d)", n_groups,
                  MAX_GROUPS);
    if (!aligned16(u_v)) return fail(PALU_EINVAL, "u_v must be 16-byte aligned");
  } else {
    if (hpg != 1) return fail(PALU_EINVAL, "grouped V latent (heads_per_group %d) needs u_v", hpg);
    if (head_dim_v != r_v)
      return fail(PALU_EINVAL, "head_dim_v %d must equal the V latent width %d on the absorbed-V path", head_dim_v, r_v);
  }
  if (cs_dtype != PALU_DTYPE_F32 && cs_dtype != PALU_DTYPE_BF16) return fail(PALU_EINVAL, "cs_tab dtype must be fp32 or bf16");
  const int out_tiled = (out_dtype & PALU_OUT_TILED_ROWS) ? 1 : 0;
  out_dtype &= ~PALU_OUT_TILED_ROWS;
  if (out_dtype != PALU_DTYPE_F32 && out_dtype != PALU_DTYPE_BF16) return fail(PALU_EINVAL, "output dtype must be fp32 or bf16");
  if (out_tiled && (batch > 64 || out_dtype != PALU_DTYPE_BF16 || ((long long)n_q * head_dim_v) % 32 != 0))
    return fail(PALU_EINVAL, "a tiled-rows output needs batch <= 64, bf16 and n_q * head_dim_v a multiple of 32");
  if (int rc = check_layout(cache_layout, seq_len, who)) return rc;
  if (!aligned16(q) || !aligned16(k_latent) || !aligned16(v_latent) || !aligned16(w_rot) || !aligned16(cs_tab))
    return fail(PALU_EINVAL, "q, k_latent, v_latent, w_rot and cs_tab must be 16-byte aligned");
  if ((long long)batch * n_kv > 65535) return fail(PALU_EUNSUPPORTED, "batch * n_kv = %d exceeds the grid limit", batch * n_kv);
  if (group_ranks != nullptr) {
    if (n_groups > MAX_GROUPS)
      return fail(PALU_EUNSUPPORTED, "group_ranks: %d latent groups (this build takes per-group ranks for up to %d)",
                  n_groups, MAX_GROUPS);
    for (int g = 0; g < 2 * n_groups; ++g) {
      const int r = group_ranks[g], top = g < n_groups ? r_k : r_v;
      if (r < 32 || r > top || r % 32 != 0)
        return fail(PALU_EINVAL, "group_ranks[%d] = %d: a group's %s rank must be a multiple of 32 in 32..%d", g, r,
                    g < n_groups ? "K" : "V", top);
      if (u_v == nullptr && r != top)
        return fail(PALU_EUNSUPPORTED, "group_ranks below the cache width need grouped latents with u_v; the "
                                       "per-head (absorbed-V) kernels read whole latent rows");
    }
  }

  memset(&a, 0, sizeof(a));
  for (int g = 0; g < MAX_GROUPS; ++g) {
    a.grk[g] = (short)(group_ranks != nullptr && g < n_groups ? group_ranks[g] : r_k);
    a.grv[g] = (short)(group_ranks != nullptr && g < n_groups ? group_ranks[n_groups + g] : r_v);
  }
  a.grp_lo = 0;
  a.grp_cnt = n_groups;
  a.rk_eff = r_k;
  a.q = static_cast<const __bf16*>(q);
  a.k = static_cast<const __bf16*>(k_latent);
  a.v = static_cast<const __bf16*>(v_latent);
  a.w_rot = static_cast<const __bf16*>(w_rot);
  a.cs = cs_tab;
  a.cur_pos = cur_pos;
  a.out = out;
  a.ws = static_cast<float*>(workspace);
  a.ws_bytes = workspace_bytes;
  a.B = batch; a.n_q = n_q; a.n_kv = n_kv; a.rep = n_q / n_kv; a.hpg = hpg; a.S = seq_len; a.cs_rows = cs_rows;
  a.deterministic = deterministic ? 1 : 0;
  a.out_tiled = out_tiled;
  a.grouped_streams = grouped_streams;
  a.qscale = scale * 1.4426950408889634f;
  a.u_v = static_cast<const __bf16*>(u_v);
  a.rk = r_k;
  a.rv = r_v;
  return PALU_OK;
}

int sdpa_dispatch(const DecodeArgs& a, bool paged, int cache_layout, int r_k, int r_v, int cs_dtype, int out_dtype,
                  hipStream_t stream) {
  // compact grouped caches use the tiled orders (sdpa_setup records them as grouped_streams)
  const bool tiled = cache_layout == PALU_LAYOUT_TILED || cache_layout == PALU_LAYOUT_TILED_GROUPED;
  if (a.u_v != nullptr) {
    if (paged) return fail(PALU_EUNSUPPORTED, "u_v: the in-kernel V rebuild is not built for paged caches");
    // Each group's stream: padded caches (tiled, or the reference's row-major [B, n_groups, S, r]) hold
    // every group at r_k / r_v columns, compact ones at the group's own ranks, one group after another
    // within a row.
    DecodeArgs ag = a;
    const int n_groups = a.n_kv / a.hpg;
    long long ok = 0, ov = 0;
    for (int g = 0; g < n_groups; ++g) {
      ag.gkw[g] = (short)(a.grouped_streams ? a.grk[g] : r_k);
      ag.gvw[g] = (short)(a.grouped_streams ? a.grv[g] : r_v);
      ag.gko[g] = ok;
      ag.gvo[g] = ov;
      ok += (long long)a.S * ag.gkw[g];
      ov += (long long)a.S * ag.gvw[g];
    }
    ag.k_sb = ok;
    ag.v_sb = ov;
    return dispatch_glrd(ag, !tiled, cs_dtype, out_dtype, stream);
  }
  if (tiled && r_k % 32 != 0)   // K rows ending in a half tile: their own translation units
    return paged ? dispatch_latent_tiled_paged_k16(a, r_k, r_v, cs_dtype, out_dtype, stream)
                 : dispatch_latent_tiled_k16(a, r_k, r_v, cs_dtype, out_dtype, stream);
  if (paged)
    return tiled ? dispatch_latent_tiled_paged(a, r_k, r_v, cs_dtype, out_dtype, stream)
                 : dispatch_latent_rows_paged(a, r_k, r_v, cs_dtype, out_dtype, stream);
  return tiled ? dispatch_latent_tiled(a, r_k, r_v, cs_dtype, out_dtype, stream)
               : dispatch_latent_rows(a, r_k, r_v, cs_dtype, out_dtype, stream);
}

int flash_setup(DecodeArgs& a, const void* q, const void* k, const void* v, const int32_t* cur_pos, void* out,
                float scale, int batch, int n_q, int n_kv, int seq_len, int head_dim_v, int out_dtype, int cache_layout,
                int deterministic, void* workspace, size_t workspace_bytes, const char* who) {
  if (!q || !k || !v || !cur_pos || !out) return fail(PALU_EINVAL, "%s: a required tensor pointer is null", who);
  if (batch <= 0 || n_q <= 0 || n_kv <= 0 || seq_len <= 0)
    return fail(PALU_EINVAL, "%s: batch, head counts and seq_len must be positive", who);
  if (n_q % n_kv != 0 || n_q / n_kv > 16)
    return fail(PALU_EINVAL, "KV head count %d must divide the %d query heads with at most 16 query heads per KV head", n_kv, n_q);
  if (out_dtype != PALU_DTYPE_F32 && out_dtype != PALU_DTYPE_BF16) return fail(PALU_EINVAL, "output dtype must be fp32 or bf16");
  if (int rc = check_layout(cache_layout, seq_len, who)) return rc;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v)) return fail(PALU_EINVAL, "q, k and v must be 16-byte aligned");
  if ((long long)batch * n_kv > 65535) return fail(PALU_EUNSUPPORTED, "batch * n_kv = %d exceeds the grid limit", batch * n_kv);
  memset(&a, 0, sizeof(a));
  a.q = static_cast<const __bf16*>(q);
  a.k = static_cast<const __bf16*>(k);
  a.v = static_cast<const __bf16*>(v);
  a.cur_pos = cur_pos;
  a.out = out;
  a.ws = static_cast<float*>(workspace);
  a.ws_bytes = workspace_bytes;
  a.B = batch; a.n_q = n_q; a.n_kv = n_kv; a.rep = n_q / n_kv; a.hpg = 1; a.S = seq_len; a.cs_rows = 0;
  a.out_tiled = 0;
  a.deterministic = deterministic ? 1 : 0;
  a.qscale = scale * 1.4426950408889634f;
  return PALU_OK;
}

// Scratch of palu_sdpa_decode_noalloc: a static device array, one copy per GPU the library runs on. Host
// code never uses the array's name as an address: its device address comes from hipGetSymbolAddress,
// once per device with that device current, and is kept per device.
__device__ __align__(256) unsigned char scratch[PALU_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;

int scratch_of_current_device(void** addr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(PALU_EHIP, "palu_sdpa_decode_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(PALU_EUNSUPPORTED, "palu_sdpa_decode_noalloc: device %d (this build keeps scratch for %d)", dev,
                kMaxDevices);
  void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr)
        return fail(PALU_EHIP, "palu_sdpa_decode_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                    hipGetErrorString(e));
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *addr = p;
  return PALU_OK;
}

}  // namespace

namespace palu {

int check_qkv_epi(const QkvEpi& e, int batch, int ncols, const void* src, const char* who) {
  if (!src || !e.pos || !e.cos_t || !e.sin_t || !e.q_out) return fail(PALU_EINVAL, "%s: a required pointer is null", who);
  if (batch < 1 || e.nh < 1 || e.table_rows < 1 || ncols <= 0 || ncols % 8)
    return fail(PALU_EINVAL, "%s: batch = %d, n_heads = %d, table_rows = %d, ncols = %d (multiple of 8)", who, batch,
                e.nh, e.table_rows, ncols);
  if (e.k_layout == PALU_LAYOUT_TILED_V || e.v_layout == PALU_LAYOUT_TILED)
    return fail(PALU_EINVAL, "%s: K caches are PALU_LAYOUT_ROWS or PALU_LAYOUT_TILED, V caches ROWS or TILED_V", who);
  if (int rc = check_append(e.kc, src, e.pos, batch, e.G, e.S, e.k_w, e.k_layout, who)) return rc;
  if (int rc = check_append(e.vc, src, e.pos, batch, e.G, e.S, e.v_w, e.v_layout, who)) return rc;
  if (!aligned16(e.q_out)) return fail(PALU_EINVAL, "%s: 16-byte alignment required", who);
  if (e.k_rope && e.k_w != HD) return fail(PALU_EINVAL, "%s: a rotated K slice is one %d-wide head, got %d", who, HD, e.k_w);
  if ((long long)e.nh * HD > ncols || e.k_off < 0 || e.v_off < 0 || e.k_gs < 0 || e.v_gs < 0 || e.k_off % 8 ||
      e.v_off % 8 || e.k_gs % 8 || e.v_gs % 8 ||
      (long long)e.k_off + (long long)(e.G - 1) * e.k_gs + e.k_w > ncols ||
      (long long)e.v_off + (long long)(e.G - 1) * e.v_gs + e.v_w > ncols)
    return fail(PALU_EINVAL, "%s: the q, K and V column ranges must lie inside the %d columns, on multiples of 8", who,
                ncols);
  return PALU_OK;
}

}  // namespace palu

extern "C" {

const char* palu_last_error(void) { return palu::g_err; }

int palu_abi_version(void) { return PALU_ABI_VERSION; }

size_t palu_decode_workspace_bytes(int batch, int n_kv, int seq_len, int head_dim_v) {
  if (batch <= 0 || n_kv <= 0 || seq_len <= 0 || head_dim_v <= 0) return 0;
  // One partial slot per workgroup of the length-aware plan (none when the items fill whole chip-fills).
  (void)seq_len;
  return decode_ws_bytes(batch * n_kv, head_dim_v);
}

size_t palu_glrd_workspace_bytes(int batch, int n_q, int n_kv, int n_groups, int seq_len, int r_v) {
  return glrd_workspace_bytes(batch, n_q, n_kv, n_groups, seq_len, r_v);
}

int palu_sdpa_decode(const void* q, const void* k_latent, const void* w_rot, const void* cs_tab, const void* v_latent,
                     int head_dim_v, const int32_t* cur_pos, void* out, const float* rot_step, const void* trans_mat,
                     const void* u_v, const int32_t* group_ranks, float scale, int heads_per_core, int rot_mode,
                     int table_mcast, int k_chunk,
                     int batch, int n_q, int n_kv, int n_groups, int seq_len, int r_k, int r_v, int w_rot_width,
                     int cs_rows, int cs_cols, int cs_dtype, int out_dtype, int cache_layout, int deterministic,
                     void* workspace, size_t workspace_bytes, hipStream_t stream) {
  palu::g_err[0] = 0;
  (void)table_mcast;
  DecodeArgs a;
  if (int rc = sdpa_setup(a, q, k_latent, w_rot, cs_tab, v_latent, head_dim_v, cur_pos, out, rot_step, trans_mat, u_v,
                          group_ranks, scale, heads_per_core, rot_mode, k_chunk, batch, n_q, n_kv, n_groups, seq_len, r_k, r_v,
                          w_rot_width, cs_rows, cs_cols, cs_dtype, out_dtype, cache_layout, deterministic, workspace,
                          workspace_bytes, "palu_sdpa_decode"))
    return rc;
  a.k_sg = (long long)seq_len * r_k;
  a.k_sb = a.k_sg * n_groups;
  a.v_sg = (long long)seq_len * r_v;
  a.v_sb = a.v_sg * n_groups;
  return sdpa_dispatch(a, false, cache_layout, r_k, r_v, cs_dtype, out_dtype, stream);
}

int palu_sdpa_decode_noalloc(const void* q, const void* k_latent, const void* w_rot, const void* cs_tab,
                             const void* v_latent, int head_dim_v, const int32_t* cur_pos, void* out,
                             const float* rot_step, const void* trans_mat, const void* u_v,
                             const int32_t* group_ranks, float scale,
                             int heads_per_core, int rot_mode, int table_mcast, int k_chunk, int batch, int n_q,
                             int n_kv, int n_groups, int seq_len, int r_k, int r_v, int w_rot_width, int cs_rows,
                             int cs_cols, int cs_dtype, int out_dtype, int cache_layout, int deterministic,
                             hipStream_t stream) {
  palu::g_err[0] = 0;
  (void)table_mcast;
  DecodeArgs a;
  // The envelope first (same checks and messages as palu_sdpa_decode), with the scratch size standing in
  // for the workspace; nothing touches the HIP runtime before the shapes are known to fit.
  if (int rc = sdpa_setup(a, q, k_latent, w_rot, cs_tab, v_latent, head_dim_v, cur_pos, out, rot_step, trans_mat, u_v,
                          group_ranks, scale, heads_per_core, rot_mode, k_chunk, batch, n_q, n_kv, n_groups, seq_len, r_k, r_v,
                          w_rot_width, cs_rows, cs_cols, cs_dtype, out_dtype, cache_layout, deterministic, nullptr,
                          PALU_NOALLOC_SCRATCH_BYTES, "palu_sdpa_decode_noalloc"))
    return rc;
  const size_t need = u_v != nullptr ? glrd_workspace_bytes(batch, n_q, n_kv, n_groups, seq_len, r_v)
                                     : decode_ws_bytes(batch * n_kv, head_dim_v);
  if (need > PALU_NOALLOC_SCRATCH_BYTES)
    return fail(PALU_EUNSUPPORTED, "palu_sdpa_decode_noalloc: these shapes need %zu bytes of scratch, more than the "
                                   "%zu of the static array; call palu_sdpa_decode with a workspace", need,
                (size_t)PALU_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (int rc = scratch_of_current_device(&ws)) return rc;
  a.ws = static_cast<float*>(ws);
  a.k_sg = (long long)seq_len * r_k;
  a.k_sb = a.k_sg * n_groups;
  a.v_sg = (long long)seq_len * r_v;
  a.v_sb = a.v_sg * n_groups;
  return sdpa_dispatch(a, false, cache_layout, r_k, r_v, cs_dtype, out_dtype, stream);
}

int palu_sdpa_decode_paged(const void* q, const void* k_pages, const void* w_rot, const void* cs_tab,
                           const void* v_pages, int head_dim_v, const int32_t* cur_pos, const int32_t* page_table,
                           void* out, const float* rot_step, const void* trans_mat, const void* u_v, float scale,
                           int heads_per_core, int rot_mode, int table_mcast, int k_chunk, int batch, int n_q, int n_kv,
                           int n_groups, int num_pages, int page_size, int max_pages_per_seq, int r_k, int r_v,
                           int w_rot_width, int cs_rows, int cs_cols, int cs_dtype, int out_dtype, int cache_layout,
                           int deterministic, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  palu::g_err[0] = 0;
  (void)table_mcast;
  int shift = 0;
  if (int rc = check_pages(page_table, num_pages, page_size, max_pages_per_seq, &shift, "palu_sdpa_decode_paged"))
    return rc;
  const int seq_len = max_pages_per_seq * page_size;
  DecodeArgs a;
  if (int rc = sdpa_setup(a, q, k_pages, w_rot, cs_tab, v_pages, head_dim_v, cur_pos, out, rot_step, trans_mat, u_v,
                          nullptr, scale, heads_per_core, rot_mode, k_chunk, batch, n_q, n_kv, n_groups, seq_len, r_k, r_v,
                          w_rot_width, cs_rows, cs_cols, cs_dtype, out_dtype, cache_layout, deterministic, workspace,
                          workspace_bytes, "palu_sdpa_decode_paged"))
    return rc;
  a.k_sg = (long long)page_size * r_k;
  a.k_sb = a.k_sg * n_groups;
  a.v_sg = (long long)page_size * r_v;
  a.v_sb = a.v_sg * n_groups;
  a.page_table = page_table;
  a.pt_stride = max_pages_per_seq;
  a.n_pages = num_pages;
  a.page_shift = shift;
  return sdpa_dispatch(a, true, cache_layout, r_k, r_v, cs_dtype, out_dtype, stream);
}

int palu_flash_decode(const void* q, const void* k, const void* v, const int32_t* cur_pos, void* out, float scale,
                      int batch, int n_q, int n_kv, int seq_len, int head_dim_v, int out_dtype, int cache_layout,
                      int deterministic, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  palu::g_err[0] = 0;
  DecodeArgs a;
  if (int rc = flash_setup(a, q, k, v, cur_pos, out, scale, batch, n_q, n_kv, seq_len, head_dim_v, out_dtype,
                           cache_layout, deterministic, workspace, workspace_bytes, "palu_flash_decode"))
    return rc;
  a.k_sg = (long long)seq_len * HD;
  a.k_sb = a.k_sg * n_kv;
  a.v_sg = (long long)seq_len * head_dim_v;
  a.v_sb = a.v_sg * n_kv;
  return dispatch_full(a, cache_layout == PALU_LAYOUT_TILED, false, head_dim_v, out_dtype == PALU_DTYPE_F32, stream);
}

int palu_flash_decode_paged(const void* q, const void* k_pages, const void* v_pages, const int32_t* cur_pos,
                            const int32_t* page_table, void* out, float scale, int batch, int n_q, int n_kv,
                            int num_pages, int page_size, int max_pages_per_seq, int head_dim_v, int out_dtype,
                            int cache_layout, int deterministic, void* workspace, size_t workspace_bytes,
                            hipStream_t stream) {
  palu::g_err[0] = 0;
  int shift = 0;
  if (int rc = check_pages(page_table, num_pages, page_size, max_pages_per_seq, &shift, "palu_flash_decode_paged"))
    return rc;
  const int seq_len = max_pages_per_seq * page_size;
  DecodeArgs a;
  if (int rc = flash_setup(a, q, k_pages, v_pages, cur_pos, out, scale, batch, n_q, n_kv, seq_len, head_dim_v,
                           out_dtype, cache_layout, deterministic, workspace, workspace_bytes, "palu_flash_decode_paged"))
    return rc;
  a.k_sg = (long long)page_size * HD;
  a.k_sb = a.k_sg * n_kv;
  a.v_sg = (long long)page_size * head_dim_v;
  a.v_sb = a.v_sg * n_kv;
  a.page_table = page_table;
  a.pt_stride = max_pages_per_seq;
  a.n_pages = num_pages;
  a.page_shift = shift;
  return dispatch_full(a, cache_layout == PALU_LAYOUT_TILED, true, head_dim_v, out_dtype == PALU_DTYPE_F32, stream);
}

int palu_latent_append(void* cache, const void* new_rows, const int32_t* update_idxs, int batch, int n_groups,
                       int seq_len, int width, int cache_layout, hipStream_t stream) {
  palu::g_err[0] = 0;
  if (int rc = check_append(cache, new_rows, update_idxs, batch, n_groups, seq_len, width, cache_layout,
                            "palu_latent_append"))
    return rc;
  return launch_append<false>(cache, new_rows, update_idxs, nullptr, 0, 0, batch, n_groups, seq_len, width,
                              cache_layout, stream);
}

int palu_qkv_post(const float* qkv_part, int ks, int batch, int ncols, const int32_t* pos, const float* cos_table,
                  const float* sin_table, int table_rows, int n_heads, void* q_out, void* k_cache, int k_layout,
                  int k_col_offset, int k_group_stride, int k_width, int k_rope, void* v_cache, int v_layout,
                  int v_col_offset, int v_group_stride, int v_width, int n_groups, int seq_len, hipStream_t stream) {
  palu::g_err[0] = 0;
  const char* who = "palu_qkv_post";
  if (!qkv_part) return fail(PALU_EINVAL, "%s: a required pointer is null", who);
  if (ks < 1 || ks > 64) return fail(PALU_EINVAL, "%s: ks = %d (1..64)", who, ks);
  const QkvEpi e{pos, cos_table, sin_table, table_rows, n_heads, static_cast<__bf16*>(q_out),
                 static_cast<__bf16*>(k_cache), k_layout, k_col_offset, k_group_stride, k_width, k_rope ? 1 : 0,
                 static_cast<__bf16*>(v_cache), v_layout, v_col_offset, v_group_stride, v_width, n_groups, seq_len};
  if (int rc = check_qkv_epi(e, batch, ncols, qkv_part, who)) return rc;
  const long long vecs = (long long)batch * (n_heads * (HD / 8) + n_groups * (k_width / 8) + n_groups * (v_width / 8));
  const int blocks = (int)std::min<long long>((vecs + 255) / 256, 2048);
  hipLaunchKernelGGL(palu_qkv_post_kernel, dim3(blocks), dim3(256), 0, stream, qkv_part, ks, batch, ncols, e);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(PALU_EHIP, "%s launch: %s", who, hipGetErrorString(err));
  return PALU_OK;
}

int palu_latent_append_strided(void* cache, const void* src, long long src_batch_stride, long long src_group_stride,
                               const int32_t* update_idxs, int batch, int n_groups, int seq_len, int width,
                               int cache_layout, hipStream_t stream) {
  palu::g_err[0] = 0;
  if (int rc = check_append(cache, src, update_idxs, batch, n_groups, seq_len, width, cache_layout,
                            "palu_latent_append_strided"))
    return rc;
  if (src_batch_stride < 0 || src_group_stride < 0 || src_batch_stride % 8 || src_group_stride % 8)
    return fail(PALU_EINVAL, "palu_latent_append_strided: source strides must be non-negative multiples of 8, got %lld "
                             "and %lld", src_batch_stride, src_group_stride);
  return launch_append<false>(cache, src, update_idxs, nullptr, 0, 0, batch, n_groups, seq_len, width, cache_layout,
                              stream, src_batch_stride, src_group_stride);
}

int palu_latent_append_grouped(void* cache, const void* src, long long src_batch_stride, long long src_group_stride,
                               const int32_t* update_idxs, int batch, int n_groups, int seq_len, const int32_t* widths,
                               int order, hipStream_t stream) {
  palu::g_err[0] = 0;
  if (!cache || !src || !update_idxs || !widths)
    return fail(PALU_EINVAL, "palu_latent_append_grouped: a required pointer is null");
  if (batch <= 0 || n_groups <= 0 || n_groups > MAX_GROUPS || seq_len <= 0 || seq_len % 32 != 0)
    return fail(PALU_EINVAL, "palu_latent_append_grouped: batch, 1..%d groups and seq_len (a multiple of 32) must be "
                             "positive, got %d, %d, %d", MAX_GROUPS, batch, n_groups, seq_len);
  if (order != PALU_LAYOUT_TILED && order != PALU_LAYOUT_TILED_V)
    return fail(PALU_EINVAL, "palu_latent_append_grouped: order must be PALU_LAYOUT_TILED (K tiles) or "
                             "PALU_LAYOUT_TILED_V (V tiles), got %d", order);
  if (src_batch_stride < 0 || src_group_stride < 0 || src_batch_stride % 8 || src_group_stride % 8)
    return fail(PALU_EINVAL, "palu_latent_append_grouped: source strides must be non-negative multiples of 8, got %lld "
                             "and %lld", src_batch_stride, src_group_stride);
  if (!aligned16(cache) || !aligned16(src)) return fail(PALU_EINVAL, "palu_latent_append_grouped: 16-byte alignment required");
  GroupTable t;
  long long off = 0;
  t.vec0[0] = 0;
  for (int g = 0; g < n_groups; ++g) {
    const int w = widths[g];
    if (w <= 0 || w % 16 != 0 || w > 512)
      return fail(PALU_EINVAL, "palu_latent_append_grouped: group %d width %d (a multiple of 16 up to 512)", g, w);
    t.off[g] = off;
    t.width[g] = w;
    t.vec0[g + 1] = t.vec0[g] + w / 8;
    off += (long long)seq_len * w;
  }
  const long long total = (long long)batch * t.vec0[n_groups];
  int blocks = (int)((total + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  auto* c = static_cast<__bf16*>(cache);
  auto* r = static_cast<const __bf16*>(src);
  if (order == PALU_LAYOUT_TILED)
    hipLaunchKernelGGL((palu_append_grouped_kernel<PALU_LAYOUT_TILED>), dim3(blocks), dim3(256), 0, stream, c, r,
                       src_batch_stride, src_group_stride, update_idxs, batch, n_groups, seq_len, off, t);
  else
    hipLaunchKernelGGL((palu_append_grouped_kernel<PALU_LAYOUT_TILED_V>), dim3(blocks), dim3(256), 0, stream, c, r,
                       src_batch_stride, src_group_stride, update_idxs, batch, n_groups, seq_len, off, t);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PALU_EHIP, "grouped append launch: %s", hipGetErrorString(e));
  return PALU_OK;
}

int palu_latent_append_paged(void* cache_pages, const void* new_rows, const int32_t* update_idxs,
                             const int32_t* page_table, int batch, int n_groups, int num_pages, int page_size,
                             int max_pages_per_seq, int width, int cache_layout, hipStream_t stream) {
  palu::g_err[0] = 0;
  int shift = 0;
  if (int rc = check_pages(page_table, num_pages, page_size, max_pages_per_seq, &shift, "palu_latent_append_paged"))
    return rc;
  if (int rc = check_append(cache_pages, new_rows, update_idxs, batch, n_groups, page_size, width, cache_layout,
                            "palu_latent_append_paged"))
    return rc;
  return launch_append<true>(cache_pages, new_rows, update_idxs, page_table, max_pages_per_seq, num_pages, batch,
                             n_groups, page_size, width, cache_layout, stream);
}

}  // extern "C"
