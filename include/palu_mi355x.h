/* C-ABI of the MI355X Palu fused latent flash-decode library (libpalu_mi355x.so).
 *
 * Every entry point takes raw device pointers, plain integer shapes and a hipStream_t, enqueues its
 * kernels on that stream and returns without synchronising. No entry point allocates device memory:
 * split-K partials go to a caller-provided workspace whose size palu_decode_workspace_bytes reports
 * (palu_sdpa_decode_noalloc keeps them in a static device array instead).
 * Tensors are dense row-major in the shapes given below; bf16 tensors must be 16-byte aligned.
 *
 * Return value: PALU_OK, or an error code with a message for palu_last_error() (thread-local, valid
 * until the next call on the same thread). Envelope messages carry the substrings the reference op's
 * own validation uses ("r_k", "cs_tab", "w_rot", "optional together", "Phase 1", "rot_mode must be",
 * "heads_per_group", "u_v", "head_dim_v", "heads_per_core", "KV head count", "grouped latents").
 */
#ifndef PALU_MI355X_H
#define PALU_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PALU_ABI_VERSION 14

#define PALU_OK 0
#define PALU_EINVAL 1       /* arguments outside the op's envelope */
#define PALU_EUNSUPPORTED 2 /* inside the reference envelope but not built in this library */
#define PALU_EHIP 3         /* HIP runtime error while launching */

#define PALU_DTYPE_F32 0
#define PALU_DTYPE_BF16 1
/* OR'ed into palu_sdpa_decode's out_dtype (bf16, batch <= 64): the output [batch, n_q * head_dim_v] is
 * written in the 64-row tiled activation layout that palu_linear_tiled reads with x_tiled = 1 (the next
 * projection of the decode step) instead of row-major. No counterpart in the reference op. */
#define PALU_OUT_TILED_ROWS 0x100

/* Cache layouts. ROWS: the reference's logical [B, G, S, width] row-major tensor. The tiled layouts
 * hold the same values with every 32-position block stored as (width / 16) tiles of 1 KB (64 slots of
 * 8 bf16) in the operand order of the kernel's MFMAs (g < 4, n < 16, c < 2):
 *   K-tile order (K latents, full K): tile c * (width/32) + kb, slot 16*g + n holds width-index
 *     32*kb + 8*g .. +7 of block position 8*(n/4) + 4*c + n%4. A width that is an odd multiple of 16
 *     (K latents of the per-head path) ends each half-block c (16 * width elements from c * 16 * width)
 *     in a 512-byte half tile: slot 16*g + n holds the 4 width-indices 32*(width/32) + 4*g .. +3;
 *   V-tile order (V latents, full V): tile mt, slot 16*g + m holds block positions 8*g .. 8*g+7 of
 *     width-index 16*mt + m.
 * A decode call with PALU_LAYOUT_TILED reads K caches in K-tile order and V caches in V-tile order;
 * the append call names the order of the cache it writes. S must be a multiple of 32 when tiled. */
#define PALU_LAYOUT_ROWS 0
#define PALU_LAYOUT_TILED 1   /* decode: K-tile K, V-tile V; append: K-tile order */
#define PALU_LAYOUT_TILED_V 2 /* append: V-tile order */
/* decode with u_v and group_ranks: grouped latents stored compactly, every group at its own ranks (K-tile
 * order for K, V-tile order for V); row b's group streams lie one after another, group g starting at
 * element b * S * sum(ranks) + S * (sum of the ranks of groups 0 .. g-1). No counterpart in the
 * reference, which pads every group to the layer's widest (convert.py:178). */
#define PALU_LAYOUT_TILED_GROUPED 3

#define PALU_ROT_LEGACY 0
#define PALU_ROT_PACK 1
#define PALU_ROT_DST 2

typedef struct ihipStream_t* palu_stream_t; /* the same handle as hipStream_t */

/* Message of the last failed call on this thread ("" after a successful one). */
const char* palu_last_error(void);

/* PALU_ABI_VERSION of the loaded library. */
int palu_abi_version(void);

/* Bytes of workspace palu_sdpa_decode / palu_flash_decode need for these shapes (0 when the
 * sequence is not split across workgroups). head_dim_v is the output width of the call. It holds the
 * split items' fp32 partials and one 8-byte chunk counter per (row, KV head); the launch merges the
 * partials itself and needs no particular contents on entry (counters of other calls count as zero).
 * Calls that share a workspace must be ordered on one stream. */
size_t palu_decode_workspace_bytes(int batch, int n_kv, int seq_len, int head_dim_v);

/* Bytes of workspace palu_sdpa_decode needs with u_v (grouped latents, in-kernel V rebuild): the fp32
 * scores ([B, n_q, S]) plus the per-split latent PV partials. The
 * grouped path runs three kernels on the stream and passes data between them through this buffer.
 * No counterpart in the reference (its op keeps these in device L1); needed because the MI355X path
 * splits the op into passes. */
size_t palu_glrd_workspace_bytes(int batch, int n_q, int n_kv, int n_groups, int seq_len, int r_v);

/* Fused latent flash-decode. Replaces ttnn.transformer.palu_sdpa_decode, the op PaluAttention's decode
 * branch calls (palu_tt/attention.py:632-639; interface in
 * docs/superpowers/specs/2026-09-10-palu-tt-stage2-design.md:47-81 and, for u_v / heads_per_core,
 * docs/superpowers/specs/2026-09-12-palu-tt-stage2b-design.md:80-139; fp32 semantics
 * palu_tt/fused.py:82-107).
 *
 *   q        [B, n_q, 128] bf16      query, already rotated at its own position (cur_pos[b])
 *   k_latent [B, n_groups, S, r_k]   bf16 K latent cache
 *   w_rot    [n_kv, r_k, 256] bf16   [u_k | u_k T] per KV head, u_k in Meta head order
 *   cs_tab   [cs_rows, 256]          [cos | sin] per position, Meta-interleaved; fp32 or bf16
 *   v_latent [B, n_groups, S, r_v]   bf16 V latent cache (absorbed V: attended over directly)
 *   r_k, r_v                         multiples of 32 (ROWS), or of 16 with PALU_LAYOUT_TILED on the
 *                                    per-head path (no u_v); the kernels are built for 32 .. 128
 *   cur_pos  [B] int32 (device)      inclusive last valid position of each row
 *   out      [B, n_q, head_dim_v]    fp32 or bf16
 *   cache_layout                     PALU_LAYOUT_ROWS or PALU_LAYOUT_TILED for both latent caches
 *   deterministic                    0: the waves of a workgroup take 32-position blocks from a shared
 *                                    counter (fastest; which wave sums which block varies, so results
 *                                    differ between calls at the bf16 rounding of the probabilities);
 *                                    1: fixed block order, bit-reproducible
 *   seq_len                          at most 65536
 *   rot_step, trans_mat              the reference's Phase 2 constants; optional together. They are
 *                                    validated as the reference does and otherwise unused: this kernel
 *                                    always rotates block-relative (32 positions) from cs_tab.
 *   u_v      [n_kv, r_v, 128] bf16   optional: in-kernel V rebuild (G-LRD). The output is then
 *                                    softmax(q K^T) (v_latent u_v[h]), 128 wide (head_dim_v == 128);
 *                                    r_k and r_v in 32 .. 512 (multiples of 32), caches in
 *                                    PALU_LAYOUT_ROWS (the reference's [B, n_groups, S, r] call,
 *                                    tests/test_palu_sdpa_device.py:245-258), PALU_LAYOUT_TILED or
 *                                    PALU_LAYOUT_TILED_GROUPED; at most 32 latent groups; not built
 *                                    for the paged entry point (PALU_EUNSUPPORTED)
 *   group_ranks [2 * n_groups] int32 (host memory, may be NULL)
 *                                    with u_v: each latent group's own ranks, K ranks then V ranks,
 *                                    multiples of 32 up to r_k / r_v. The caches keep r_k / r_v columns
 *                                    per group (the reference pads every group to the layer's widest);
 *                                    the kernels read and multiply only a group's own columns, so the
 *                                    padding is never touched. NULL: every group at r_k / r_v. Without
 *                                    u_v every entry must equal r_k / r_v (PALU_EUNSUPPORTED otherwise).
 *                                    No counterpart in the reference's op interface.
 *   scale                            softmax scale (the reference passes head_dim^-0.5)
 *   heads_per_core, rot_mode, table_mcast, k_chunk
 *                                    the reference's Tensix work-split switches; validated, and
 *                                    otherwise without effect on MI355X (k_chunk 0 = default)
 * Head h of q attends KV head h / (n_q / n_kv); KV head j reads latent group j / (n_kv / n_groups).
 */
int palu_sdpa_decode(const void* q, const void* k_latent, const void* w_rot, const void* cs_tab, const void* v_latent,
                     int head_dim_v, const int32_t* cur_pos, void* out, const float* rot_step, const void* trans_mat,
                     const void* u_v, const int32_t* group_ranks, float scale, int heads_per_core, int rot_mode,
                     int table_mcast, int k_chunk,
                     int batch, int n_q, int n_kv, int n_groups, int seq_len, int r_k, int r_v, int w_rot_width,
                     int cs_rows, int cs_cols, int cs_dtype, int out_dtype, int cache_layout, int deterministic,
                     void* workspace, size_t workspace_bytes, palu_stream_t stream);

/* Bytes of the static device scratch array behind palu_sdpa_decode_noalloc (one per GPU). */
#define PALU_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* palu_sdpa_decode without a workspace argument, allocating nothing. No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The scratch memory the kernels need (split partials of the
 * length-aware plan; the grouped-latent path's scores and PV partials) lives in a static device array of
 * PALU_NOALLOC_SCRATCH_BYTES per GPU that the library holds until the process ends; the array of the
 * current device (hipGetDevice) is used, so the stream must belong to that device. Shapes whose scratch
 * need (palu_decode_workspace_bytes, or palu_glrd_workspace_bytes with u_v) exceeds it are rejected with
 * PALU_EUNSUPPORTED before anything is launched. Every call on one GPU shares that GPU's array: calls
 * ordered on one stream are safe; calls that overlap on one GPU (several streams or host threads) race.
 * Every other argument, the envelope and the error messages are those of palu_sdpa_decode. */
int palu_sdpa_decode_noalloc(const void* q, const void* k_latent, const void* w_rot, const void* cs_tab,
                             const void* v_latent, int head_dim_v, const int32_t* cur_pos, void* out,
                             const float* rot_step, const void* trans_mat, const void* u_v,
                             const int32_t* group_ranks, float scale,
                             int heads_per_core, int rot_mode, int table_mcast, int k_chunk, int batch, int n_q,
                             int n_kv, int n_groups, int seq_len, int r_k, int r_v, int w_rot_width, int cs_rows,
                             int cs_cols, int cs_dtype, int out_dtype, int cache_layout, int deterministic,
                             palu_stream_t stream);

/* Paged fused latent flash-decode: palu_sdpa_decode over caches held in fixed-size pages. The reference
 * keeps contiguous per-row caches (palu_tt/attention.py:86, 274-283); paging follows ttnn's paged decode
 * interface (paged_scaled_dot_product_attention_decode: page pools plus a per-row page table).
 *   k_pages     [num_pages, n_groups, page_size, r_k] bf16 pool (row-major, or tiled per 32-position
 *               block inside each page when cache_layout is PALU_LAYOUT_TILED)
 *   v_pages     [num_pages, n_groups, page_size, r_v] bf16 pool, same layout
 *   page_table  [batch, max_pages_per_seq] int32 (device): position p of row b lives on page
 *               page_table[b][p / page_size], row p % page_size. Ids are clamped into [0, num_pages).
 *   page_size   a power of two in 32..4096; the logical length is max_pages_per_seq * page_size
 *               (at most 65536) and cs_tab needs that many rows.
 * Every other argument as for palu_sdpa_decode; palu_decode_workspace_bytes takes the logical length. */
int palu_sdpa_decode_paged(const void* q, const void* k_pages, const void* w_rot, const void* cs_tab,
                           const void* v_pages, int head_dim_v, const int32_t* cur_pos, const int32_t* page_table,
                           void* out, const float* rot_step, const void* trans_mat, const void* u_v, float scale,
                           int heads_per_core, int rot_mode, int table_mcast, int k_chunk, int batch, int n_q, int n_kv,
                           int n_groups, int num_pages, int page_size, int max_pages_per_seq, int r_k, int r_v,
                           int w_rot_width, int cs_rows, int cs_cols, int cs_dtype, int out_dtype, int cache_layout,
                           int deterministic, void* workspace, size_t workspace_bytes, palu_stream_t stream);

/* Stock flash-decode over full, already-rotated K and a V cache of width head_dim_v. Replaces
 * ttnn.transformer.scaled_dot_product_attention_decode (head_dim_v == 128) and
 * ttnn.transformer.flash_multi_latent_attention_decode (head_dim_v == r_v), the two ops the reference's
 * non-fused decode path calls (palu_tt/attention.py:703-706; tests/test_palu_sdpa_device.py:58-65,
 * 238-241). It is also the full-KV comparator for the fused op.
 *   q [B, n_q, 128] bf16, k [B, n_kv, S, 128] bf16, v [B, n_kv, S, head_dim_v] bf16,
 *   cur_pos [B] int32 (device), out [B, n_q, head_dim_v] fp32 or bf16; cache_layout and deterministic
 *   as for palu_sdpa_decode. */
int palu_flash_decode(const void* q, const void* k, const void* v, const int32_t* cur_pos, void* out, float scale,
                      int batch, int n_q, int n_kv, int seq_len, int head_dim_v, int out_dtype, int cache_layout,
                      int deterministic, void* workspace, size_t workspace_bytes, palu_stream_t stream);

/* Stock flash-decode over paged full K / V pools ([num_pages, n_kv, page_size, 128] and
 * [num_pages, n_kv, page_size, head_dim_v]); replaces ttnn.transformer.paged_scaled_dot_product_attention_decode.
 * Paging arguments as for palu_sdpa_decode_paged, the rest as for palu_flash_decode. */
int palu_flash_decode_paged(const void* q, const void* k_pages, const void* v_pages, const int32_t* cur_pos,
                            const int32_t* page_table, void* out, float scale, int batch, int n_q, int n_kv,
                            int num_pages, int page_size, int max_pages_per_seq, int head_dim_v, int out_dtype,
                            int cache_layout, int deterministic, void* workspace, size_t workspace_bytes,
                            palu_stream_t stream);

/* Latent append: cache[b, g, update_idxs[b], :] = new_rows[b, g, :] for every row whose index lies in
 * [0, seq_len) (other rows are skipped). Replaces ttnn.experimental.paged_update_cache on the latent
 * caches (palu_tt/attention.py:622-623).
 *   cache [B, n_groups, S, width] bf16, new_rows [B, n_groups, width] bf16, update_idxs [B] int32
 *   (device), width a multiple of 8 (of 32 for a tiled cache); cache_layout PALU_LAYOUT_ROWS,
 *   PALU_LAYOUT_TILED (a K cache) or PALU_LAYOUT_TILED_V (a V cache). */
int palu_latent_append(void* cache, const void* new_rows, const int32_t* update_idxs, int batch, int n_groups,
                       int seq_len, int width, int cache_layout, palu_stream_t stream);

/* Paged latent append: row b goes to page page_table[b][update_idxs[b] / page_size] of the pool
 * [num_pages, n_groups, page_size, width], row update_idxs[b] % page_size (rows whose position is past
 * max_pages_per_seq * page_size or whose page id is outside the pool are skipped). Replaces
 * ttnn.experimental.paged_update_cache with a page table (palu_tt/attention.py:622-623 is its
 * contiguous use). Layouts as for palu_latent_append. */
int palu_latent_append_paged(void* cache_pages, const void* new_rows, const int32_t* update_idxs,
                             const int32_t* page_table, int batch, int n_groups, int num_pages, int page_size,
                             int max_pages_per_seq, int width, int cache_layout, palu_stream_t stream);

/* ---- Decoder-step helpers ---------------------------------------------------------------------------
 * No counterpart in the reference's op interface. palu_tt.attention and palu_tt.model use them to fuse
 * the elementwise work around the decode op, which the reference runs as separate ttnn ops
 * (palu_tt/attention.py:585-733: rotary_embedding_llama, the latent slices, paged_update_cache; the
 * tt_transformers decoder's RMSNorm and SwiGLU MLP). bf16 tensors, fp32 arithmetic. */

/* Latent append from a strided source: cache[b, g, update_idxs[b], :] = src[b * src_batch_stride +
 * g * src_group_stride + 0 .. width - 1] (element strides, multiples of 8), e.g. the latent columns of
 * a fused QKV projection's output; everything else as palu_latent_append. */
int palu_latent_append_strided(void* cache, const void* src, long long src_batch_stride, long long src_group_stride,
                               const int32_t* update_idxs, int batch, int n_groups, int seq_len, int width,
                               int cache_layout, palu_stream_t stream);

/* Latent append into grouped latents stored compactly (PALU_LAYOUT_TILED_GROUPED): group g's stream of
 * row b (offsets as that layout says, widths[g] wide: host memory, multiples of 16 up to 512) gets at
 * position update_idxs[b] the first widths[g] values of src[b * src_batch_stride + g * src_group_stride
 * ..], in K-tile (order = PALU_LAYOUT_TILED) or V-tile order (PALU_LAYOUT_TILED_V). seq_len a multiple of
 * 32, at most 32 groups. No counterpart in the reference (its caches are padded to the widest group). */
int palu_latent_append_grouped(void* cache, const void* src, long long src_batch_stride, long long src_group_stride,
                               const int32_t* update_idxs, int batch, int n_groups, int seq_len, const int32_t* widths,
                               int order, palu_stream_t stream);

/* The decode step's QKV epilogue in one launch, from the fp32 split partials [ks, batch, ncols] of the
 * QKV projection (palu_linear_tiled with PALU_LINEAR_F32_PARTIALS), summed in slice order: q_out
 * [batch, n_heads, 128] = the first n_heads 128-wide heads rotated at pos[b] (as palu_rope_rows), and for
 * every latent group g the K slice (columns k_col_offset + g * k_group_stride, k_width wide; rotated as
 * well when k_rope, then k_width must be 128) and the V slice (v_col_offset + g * v_group_stride, v_width
 * wide) appended at pos[b] to k_cache / v_cache (as palu_latent_append_strided; K caches ROWS or TILED,
 * V caches ROWS or TILED_V). Column offsets and strides multiples of 8. */
int palu_qkv_post(const float* qkv_part, int ks, int batch, int ncols, const int32_t* pos, const float* cos_table,
                  const float* sin_table, int table_rows, int n_heads, void* q_out, void* k_cache, int k_layout,
                  int k_col_offset, int k_group_stride, int k_width, int k_rope, void* v_cache, int v_layout,
                  int v_col_offset, int v_group_stride, int v_width, int n_groups, int seq_len, palu_stream_t stream);

/* Per row of [rows, dim]: h = x + res, rounded to bf16 and stored to h_out when h_out is not NULL;
 * y_out = h * rsqrt(mean(h^2) + eps) * weight. dim a multiple of 8, at most 8192. The residual input is
 * res (bf16 [rows, dim]), or res_part (fp32 [res_ks, rows, dim]: the split partials of a projection's
 * PALU_LINEAR_F32_PARTIALS output, summed here), or neither (h = x). y_tiled = 1 writes y_out in the
 * 64-row tiled activation layout that palu_linear_tiled reads with x_tiled = 1 (rows <= 64, dim a
 * multiple of 32; the buffer holds 64 rows, those past `rows` untouched). */
int palu_rmsnorm(const void* x, const void* res, const float* res_part, int res_ks, void* h_out, void* y_out,
                 const void* weight, int rows, int dim, float eps, int y_tiled, palu_stream_t stream);

/* out[r][f] = silu(gu[r][f]) * gu[r][ffn + f] for gu [rows, 2 ffn], out [rows, ffn]; ffn a multiple of 8.
 * out_tiled = 1 writes out in the 64-row tiled activation layout (rows <= 64, ffn a multiple of 32). */
int palu_swiglu(const void* gu, void* out, int rows, int ffn, int out_tiled, palu_stream_t stream);

/* Greedy sampling: out[r] = index of the largest value of row r of x (bf16, rows of n values, row stride
 * ld elements: ld >= n, a multiple of 8), the first one among equal maxima and NaN above every number
 * (torch.argmax's result). No counterpart in the reference's op interface: its generation loop takes
 * the argmax of the host-side logits (generate.py:53-62); this keeps the decode step's greedy pick in
 * the same HIP graph as the step. */
int palu_argmax_rows(const void* x, long long ld, int rows, int n, int64_t* out, palu_stream_t stream);

/* Meta-interleaved RoPE of `heads` 128-wide heads per row at the row's position:
 * dst[b, h, :] = rotate(src[b * src_row_stride + h * 128 .. +127], pos[b]), pairs (2i, 2i+1) ->
 * (x0 c - x1 s, x1 c + x0 s) with c = cos_table[p][2i], s = sin_table[p][2i] (fp32 [table_rows, 128],
 * fused.cos_sin_tables). Positions outside the table are clamped into it. dst is [rows, heads, 128]. */
int palu_rope_rows(const void* src, long long src_row_stride, void* dst, const int32_t* pos, const float* cos_table,
                   const float* sin_table, int table_rows, int rows, int heads, palu_stream_t stream);

/* Output modes of palu_linear_tiled. */
#define PALU_LINEAR_BF16 0          /* y: bf16 [rows, n], rows ldy apart */
#define PALU_LINEAR_F32_PARTIALS 1  /* y: fp32 [ks, rows, n], the k slices' partial sums, not added up */
#define PALU_LINEAR_SWIGLU_TILED 2  /* y: bf16 [64, n / 2] tiled activations, silu(gate) * up (ks = 1) */

/* Decode-step projection: y[r][c] = sum_k x[r][k] w[c][k] for rows = 1..64 (bf16 in, fp32 accumulate),
 * with w [n, k] given tiled for groups of rtw row tiles (palu_tt.decoder_ops.tile_weight: 16 x 32 tiles
 * of 1 KB, lane 16 g + i of tile (rt, kt) holding w[16 rt + i][32 kt + 8 g .. +7]; row tiles in groups of
 * rtw, the last group possibly shorter, each group's tiles stored [kt][rt in group]). x is row-major with
 * rows ldx apart (x_tiled = 0; ldx >= k, a multiple of 8) or in the 64-row tiled activation layout
 * (x_tiled = 1: the same 1 KB tiles over 64 rows, stored [kt][row tile], rows past `rows` ignored;
 * palu_rmsnorm and palu_swiglu write it). n a multiple of 16, k of 32, x 16-byte aligned. rtw (1..8)
 * must be the one the weight was tiled with; ks (1..64) k slices. y_mode PALU_LINEAR_BF16: y rows ldy
 * apart (>= n, a multiple of 4); with ks > 1 the slices' fp32 partials go through a caller workspace of
 * palu_linear_workspace_bytes(rows, n, k, ks) bytes and a second launch adds them. PALU_LINEAR_F32_PARTIALS:
 * y receives the ks partial sums (no workspace, no second launch). PALU_LINEAR_SWIGLU_TILED: w holds
 * gate and up rows interleaved eight at a time (rows 16 j .. 16 j + 7 gate outputs 8 j .. 8 j + 7, rows
 * 16 j + 8 .. 16 j + 15 the up rows of the same outputs; n a multiple of 64, ks = 1) and y receives
 * silu(gate) * up as the [64, n / 2] tiled activations of the next projection.
 * palu_linear_plan suggests (rtw, ks) for a shape. The reference's counterpart is the ttnn.linear of
 * each projection of its decode step. */
int palu_linear_tiled(const void* x, long long ldx, int x_tiled, int rows, const void* w_tiled, int n, int k, void* y,
                      long long ldy, int y_mode, int rtw, int ks, void* workspace, size_t workspace_bytes,
                      palu_stream_t stream);

/* A work split (rtw, ks) for palu_linear_tiled at this shape, from a model of the busiest CU's bytes. */
int palu_linear_plan(int rows, int n, int k, int* rtw, int* ks);

/* Workspace bytes of palu_linear_tiled with ks k slices (0 for ks == 1 or invalid shapes). */
size_t palu_linear_workspace_bytes(int rows, int n, int k, int ks);

/* Greedy pick fused into the LM head: ids[r] (r < rows) = the index of the largest value of row r of
 * the bf16 result palu_linear_tiled gives with PALU_LINEAR_BF16 and ks = 1 (the same sums in the same
 * order, rounded the same way), the first one among equal maxima and NaN above every number: what
 * palu_argmax_rows returns for those logits, which are not written. x, w_tiled, n, k and rtw as in
 * palu_linear_tiled; a caller workspace of palu_linear_argmax_workspace_bytes(rows, n) bytes (16-byte
 * aligned) holds one key per row and workgroup (at most 256 workgroups, each running groups of rtw row
 * tiles). Two launches. No counterpart in the
 * reference's op interface: its generation loop takes the argmax of the host-side logits
 * (generate.py:53-62); this keeps the greedy pick in the decode step's graph without writing the 64 x
 * vocab logits and reading them back. */
int palu_linear_argmax(const void* x, long long ldx, int x_tiled, int rows, const void* w_tiled, int n, int k, int rtw,
                       int64_t* ids, void* workspace, size_t workspace_bytes, palu_stream_t stream);

/* Workspace bytes of palu_linear_argmax (0 for invalid shapes). */
size_t palu_linear_argmax_workspace_bytes(int rows, int n);

/* palu_linear_plan with at most max_ks k slices (max_ks = 1: the split for the fused epilogues below,
 * which see whole dot products). */
int palu_linear_plan_ks(int rows, int n, int k, int max_ks, int* rtw, int* ks);

/* The gate / up projection over RMS-normalised rows, in one launch: with w the interleaved gate / up
 * weight of palu_linear_tiled's SwiGLU mode whose columns carry the norm's weight (w[c][j] = w_ffn[c][j]
 * * norm_weight[j]), y_tiled [64, n / 2] receives silu(g) * u for g, u = (x w^T) * rsqrt(mean_j(x^2) +
 * eps) per row, i.e. the SwiGLU of the normalised x, the sum of squares taken over the bf16 x the
 * product reads. x, rows, w, n, k, rtw as palu_linear_tiled (one k slice; n a multiple of 64); y_tiled must
 * not overlap x (every workgroup reads all of x while others write their outputs). Replaces
 * palu_rmsnorm followed by the SwiGLU projection (the reference model's ffn_norm and w1 / w3 of its decode
 * step); no counterpart in the reference's op interface. */
int palu_linear_swiglu_rmsnorm(const void* x, long long ldx, int x_tiled, int rows, const void* w_tiled, int n, int k,
                               int rtw, float eps, void* y_tiled, palu_stream_t stream);

/* Residual update by a projection, in one launch: h[r][c] = bf16(h[r][c] + sum_k x[r][k] w[c][k]) for h
 * bf16 [rows, n] with rows ldh apart (>= n, a multiple of 4; h 8-byte aligned), and, when h_tiled is not
 * NULL, the same values in the 64-row tiled activation layout (n a multiple of 32) for the projection
 * that reads h next. x, rows, w, n, k, rtw as palu_linear_tiled (one k slice); h and h_tiled must not
 * overlap x. Replaces the output projection plus the residual add of the reference model's decode step;
 * no counterpart in the reference's op interface. */
int palu_linear_residual(const void* x, long long ldx, int x_tiled, int rows, const void* w_tiled, int n, int k,
                         int rtw, void* h, long long ldh, void* h_tiled, palu_stream_t stream);

/* The decode step's QKV projection with its epilogue in the same launch: the product y = x w^T (one k
 * slice) goes where palu_qkv_post sends its summed partials (q_out, and the K / V latent appends at
 * pos[b], arguments as palu_qkv_post with ncols = n), rounded the same way. The q heads, the K slices and
 * the V slices must not overlap (group strides at least the widths), and q_out and the caches must not
 * overlap x. The reference's counterpart is the fused QKV ttnn.linear, RoPE and paged_update_cache calls
 * of its decode step (attention.py:585-623). */
int palu_linear_qkv(const void* x, long long ldx, int x_tiled, int rows, const void* w_tiled, int n, int k, int rtw,
                    const int32_t* pos, const float* cos_table, const float* sin_table, int table_rows, int n_heads,
                    void* q_out, void* k_cache, int k_layout, int k_col_offset, int k_group_stride, int k_width,
                    int k_rope, void* v_cache, int v_layout, int v_col_offset, int v_group_stride, int v_width,
                    int n_groups, int seq_len, palu_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PALU_MI355X_H */
