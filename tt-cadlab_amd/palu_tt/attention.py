"""PaluAttention on MI355X: the reference's attention drop-in (palu_tt/attention.py:97-733) over
PyTorch-ROCm tensors and the HIP decode library.

Same construction inputs and state-dict keys as the reference (``layers.{i}.attention.wq.weight`` /
``.wo.weight`` and the converter's ``layers.{i}.attention.palu.*``, convert.palu_layer_tensors), the
same cache contents (latent rows of width r_k / r_v per head or per group, or rotated full K on the
K-fast path), and the same decode data flow (attention.py:585-733):

  decode:  x @ [wq | wk_lat | wv_lat]^T -> q, latents (one GEMM; wk_lat / wv_lat are the latent rows of
           the converter's wk_lat_pad / wv_lat_pad, a head's first r rows or a group's, without the
           zero padding to head_dim)
           RoPE on q at current_pos (Meta-interleaved) and the latents appended at current_pos, both
           straight from the GEMM output (one fused launch over the projection's split partials)
           with PaluRuntime.use_fused_k: fused latent flash-decode (palu_sdpa_decode; u_v rebuilds V
           per head for grouped latents);
           without it (the reference's default, attention.py:657-710): the naive path, which rebuilds
           K = latent @ u_k for the first recon_len positions, rotates it (prefill-mode RoPE), rebuilds
           grouped V with u_v, and runs the stock flash-decode over them;
           on the K-fast path (r_k == head_dim, per-head factors), flash-decode over the cached
           rotated K
           absorbed-V output @ the r_v rows per head of wo_fused^T (the reference pads the output to
           head_dim and multiplies the full wo_fused; the padded rows contribute zero)
  prefill: latents rebuilt to full K / V with u_k / u_v (attention.py:380-480), RoPE on q and K,
           causal SDPA, @ wo^T; the cache receives the latents (or rotated K on the fast path).

Tensors: x is [B, dim] for decode (or the reference's [1, 1, B, dim]) and [1, S, dim] / [1, 1, S, dim]
for prefill; outputs have the matching shape. The caches are ``LatentCache`` objects (the tiled layout
the kernels stream fastest) unless ``cache_layout="rows"`` is asked for.
"""
from typing import Optional

import torch
import torch.nn.functional as F

from palu_tt import decoder_ops, fused
from palu_tt.cache import GroupedLatentCache, LatentCache


def kernel_group_ranks(ranks_k, ranks_v, r_k: int, r_v: int):
    """The per-group ranks a layer hands to the fused op and its compact caches: each group's rank from the
    factor directory (config.json head_wise_ranks, any positive integer) rounded up to a multiple of 32,
    capped at the layer's padded r_k / r_v, and the widest group at exactly r_k / r_v (so the compact
    cache's logical width is the layer's). The factors are zero in the columns added (load_palu_dir pads
    every group with zeros), so the products are unchanged; the grouped-latent kernels take group ranks
    in multiples of 32."""
    def fit(ranks, top):
        out = [min(-(-int(r) // 32) * 32, top) for r in ranks]
        out[max(range(len(out)), key=out.__getitem__)] = top
        return out
    return fit(ranks_k, int(r_k)), fit(ranks_v, int(r_v))


class PaluAttention(torch.nn.Module):
    def __init__(self, mesh_device, tt_ccl, args, state_dict, weight_cache_path, layer_num, dtype=torch.bfloat16,
                 transformation_mats=None, configuration=None, paged_attention_config=None, use_paged_kv_cache=False,
                 prefetcher=None, cache_layout: str = "tiled"):
        super().__init__()
        assert paged_attention_config is None and not use_paged_kv_cache, \
            "the attention module keeps contiguous per-row caches (the paged kernels are in palu_tt.fused)"
        assert prefetcher is None, "prefetcher not supported"
        configuration = configuration if configuration is not None else args
        assert hasattr(configuration, "palu"), "attach a PaluConfig as configuration.palu"
        assert cache_layout in ("tiled", "rows")
        self.device = torch.device(mesh_device) if not isinstance(mesh_device, torch.device) else mesh_device
        self.dtype = dtype
        self.layer_num = layer_num
        self.hidden_size = configuration.dim
        self.n_heads = configuration.n_heads
        self.n_kv_heads = configuration.n_kv_heads
        self.head_dim = configuration.head_dim
        self.max_seq_len = configuration.max_seq_len
        self.max_batch_size = configuration.max_batch_size
        self.scale = self.head_dim ** -0.5
        self.palu = configuration.palu
        self.gs = int(self.palu.group_size)
        assert self.n_kv_heads % self.gs == 0, f"group size {self.gs} must divide {self.n_kv_heads} KV heads"
        self.n_groups = self.n_kv_heads // self.gs
        self.r_k = int(self.palu.rank_k[layer_num])
        self.r_v = int(self.palu.rank_v[layer_num])
        hd = self.head_dim
        # tiled caches of per-head latents take ranks in multiples of 16 (16-wide V tiles, K rows ending in a
        # half tile); row-major caches and grouped latents keep multiples of 32
        step = 16 if (cache_layout == "tiled" and self.gs == 1) else 32
        assert self.r_k % step == 0 and self.r_v % step == 0 and self.r_k <= self.gs * hd and self.r_v <= self.gs * hd, \
            f"ranks r_k = {self.r_k}, r_v = {self.r_v} must be multiples of {step}"
        # full-rank per-head factors collapse to stock K / V (reference attention.py:136-141)
        self.recon_k = self.gs > 1 or self.r_k < hd
        self.recon_v = self.gs > 1 or self.r_v < hd
        # the fused op replaces the naive rebuild only where K really is a latent (reference
        # attention.py:151); PaluRuntime() defaults to the naive path, as the reference's does
        self.use_fused_k = self.recon_k and bool(self.palu.runtime.use_fused_k)
        # grouped latents of unequal ranks (padded to rank_k / rank_v): the fused op reads only each
        # group's own columns (rounded up to the kernels' multiple of 32) when it is given the groups' ranks
        gr = self.palu.group_ranks[layer_num] if self.palu.group_ranks else None
        self.group_ranks = kernel_group_ranks(gr[0], gr[1], self.r_k, self.r_v) if (gr is not None and self.gs > 1) \
            else None
        self.cache_layout = cache_layout
        self._naive_pos = {}

        ln = f"layers.{layer_num}.attention"
        P = f"{ln}.palu"
        dev, bf = self.device, torch.bfloat16
        wq = state_dict[f"{ln}.wq.weight"]
        # the latent rows of wk_lat_pad / wv_lat_pad: group g's rows g * gs * hd .. + width (a head's
        # first r rows for group size 1, the whole head on the full-rank paths); the rest is zero padding
        self.k_width = self.r_k if self.recon_k else hd
        gw = lambda w, width: w.reshape(self.n_groups, self.gs * hd, -1)[:, :width].reshape(-1, w.shape[-1])
        wk = gw(state_dict[f"{P}.wk_lat_pad"], self.k_width)
        wv = gw(state_dict[f"{P}.wv_lat_pad"], self.r_v)
        # [nh hd + n_groups (k_width + r_v), dim]: held in the decode projection's tiled order
        # (decoder_ops.DecodeLinear); the prefill multiplies by its nn.Linear-layout copy
        self.wqkv = decoder_ops.DecodeLinear(torch.cat([wq, wk, wv], dim=0).to(dev, bf).contiguous(),
                                             self.max_batch_size, single_slice=True)
        self.wo = state_dict[f"{ln}.wo.weight"].to(dev, bf).contiguous()
        wo_fused = (state_dict[f"{P}.wo_fused"].to(dev, bf) if (self.recon_v and self.gs == 1) else self.wo)
        # decode output width per head: the absorbed-V latent (r_v) or, with u_v / stock V, head_dim; the
        # output projection keeps only those rows of wo_fused (the rest multiply the zero padding)
        self.out_width = self.head_dim if (self.gs > 1 or not self.recon_v) else self.r_v
        self.wo_out = decoder_ops.DecodeLinear(wo_fused.view(-1, self.n_heads, self.head_dim)[:, :, :self.out_width]
                                               .reshape(-1, self.n_heads * self.out_width).contiguous(),
                                               self.max_batch_size, single_slice=True)
        self.u_k = state_dict[f"{P}.u_k"].to(dev, bf).contiguous() if self.recon_k else None   # [nkv, r_k, hd]
        self.w_rot = state_dict[f"{P}.w_rot"].to(dev, bf)[None].contiguous() if self.recon_k else None
        self.u_v = state_dict[f"{P}.u_v"].to(dev, bf).contiguous() if self.recon_v else None   # [nkv, r_v, hd]

        cos, sin = fused.cos_sin_tables(hd, self.max_seq_len, configuration.rope_theta,
                                        getattr(configuration, "rope_scaling", None))
        self.cos = cos[:self.max_seq_len].to(dev).contiguous()
        self.sin = sin[:self.max_seq_len].to(dev).contiguous()
        self.cs_tab = fused.cs_table(cos, sin, self.max_seq_len)[None, None].to(dev).contiguous()

        B, S = self.max_batch_size, self.max_seq_len
        k_width = self.r_k if self.recon_k else hd
        if cache_layout == "tiled" and self.group_ranks is not None:
            # grouped latents of unequal ranks: every group stored at its own ranks (the reference pads
            # each to the widest, attention.py:274-283 with convert.py:178)
            assert S % 32 == 0, "the tiled cache holds whole 32-position blocks"
            keys = GroupedLatentCache.zeros(B, self.group_ranks[0], S, dev, "k")
            values = GroupedLatentCache.zeros(B, self.group_ranks[1], S, dev, "v")
        elif cache_layout == "tiled":
            assert S % 32 == 0, "the tiled cache holds whole 32-position blocks"
            keys = LatentCache.zeros(B, self.n_groups, S, k_width, dev, "k")
            values = LatentCache.zeros(B, self.n_groups, S, self.r_v, dev, "v")
        else:
            keys = torch.zeros(B, self.n_groups, S, k_width, dtype=bf, device=dev)
            values = torch.zeros(B, self.n_groups, S, self.r_v, dtype=bf, device=dev)
        self.layer_past = [keys, values]

    # ------------------------------------------------------------------------------------------------
    def kv_bytes_per_token(self) -> float:
        """Cache bytes per token per layer (bf16 latents), reference attention.py:352-358; compact grouped
        caches count each group at its own ranks."""
        keys, values = self.layer_past
        if isinstance(keys, GroupedLatentCache):
            return (sum(keys.ranks) + sum(values.ranks)) * 2.0
        k_width = self.r_k if self.recon_k else self.head_dim
        return self.n_groups * (k_width + self.r_v) * 2.0

    def _split(self, xqkv):
        """[..., nh hd + G (k_width + r_v)] projection output -> q [..., nh, hd], K latents [..., G, k_width]
        (the rotated-later full K heads on the full-rank path), V latents [..., G, r_v]."""
        nh, hd, G = self.n_heads, self.head_dim, self.n_groups
        k0, v0 = nh * hd, nh * hd + G * self.k_width
        q = xqkv[..., :k0].unflatten(-1, (nh, hd))
        k = xqkv[..., k0:v0].unflatten(-1, (G, self.k_width))
        v = xqkv[..., v0:].unflatten(-1, (G, self.r_v))
        return q, k, v

    def _rope(self, x, pos):
        """Meta-interleaved RoPE of x [..., heads, hd] at positions pos (broadcast over heads)."""
        return fused.apply_rope_meta(x, self.cos[pos][..., None, :], self.sin[pos][..., None, :])

    # ------------------------------------------------------------------------------------------------
    def forward_decode(self, x, current_pos, rot_mats=None, page_table=None, kv_cache=None, x_tiled=False,
                       out_partials=False, residual=None):
        """One decode step for all max_batch_size rows: QKV projection; RoPE of q (and of K on the K-fast
        path) and the latent appends from the projection's columns (in the projection's own epilogue when
        it is tiled in one k slice, else one fused launch over its split partials); the fused op (or the
        naive path, or the stock decode over rotated K); output projection over the out_width rows per
        head. With x_tiled, x is the [64, dim] tiled activation buffer (decoder_ops.rmsnorm(...,
        tiled_out=True)) holding the max_batch_size rows, and the output is [max_batch_size, dim]; with
        out_partials it is the output projection's fp32 split partials [ks, B, dim] (decoder_ops.rmsnorm's
        res_part); with residual = (h, h_tiled) the output projection adds into the residual stream h
        [B, dim] in place and writes the new h to the tiled buffer h_tiled (decoder_ops.linear_residual),
        and h is returned."""
        assert page_table is None and kv_cache is None
        if x_tiled:
            B = self.max_batch_size
            shape, x2 = (B, self.hidden_size), x
        else:
            shape = x.shape
            x2 = x.reshape(-1, self.hidden_size).to(torch.bfloat16)
            B = x2.shape[0]
        if B != self.max_batch_size:
            raise ValueError(f"decode batch {B} != max_batch_size {self.max_batch_size}")
        pos = current_pos.reshape(-1).to(self.device, torch.int32)
        assert pos.numel() == B
        nh, nkv, hd = self.n_heads, self.n_kv_heads, self.head_dim
        keys, values = self.layer_past
        kw, G = self.k_width, self.n_groups
        k0, v0 = nh * hd, nh * hd + G * kw                                  # column offsets of K and V latents
        if self.wqkv.tiled and self.wqkv.ks == 1 and not isinstance(keys, GroupedLatentCache):
            q = self.wqkv.qkv(x2, pos, self.cos, self.sin, nh, keys, k0, kw, kw, values, v0, self.r_v, self.r_v,
                              k_rope=not self.recon_k, x_tiled=x_tiled, rows=B)
        elif self.wqkv.tiled and not isinstance(keys, GroupedLatentCache):
            part = self.wqkv(x2, x_tiled=x_tiled, rows=B, mode="partials")  # [ks, B, nh hd + G (kw + r_v)] fp32
            q = decoder_ops.qkv_post(part, pos, self.cos, self.sin, nh, keys, k0, kw, kw, values, v0, self.r_v,
                                     self.r_v, k_rope=not self.recon_k)
        else:
            # bf16 projection output; compact grouped caches take their appends from its columns
            xqkv = self.wqkv(x2, x_tiled=x_tiled, rows=B) if x_tiled else self.wqkv(x2)   # [B, nh hd + G (kw + r_v)]
            q = decoder_ops.rope_rows(xqkv, nh, pos, self.cos, self.sin)     # [B, nh, hd]
            kcols, vcols = xqkv[:, k0:], xqkv[:, v0:]
            if self.recon_k:
                decoder_ops.append_from(keys, kcols, kw, kw, pos)
            else:                                                            # stock K path: rotated full K
                k_rot = decoder_ops.rope_rows(kcols, nkv, pos, self.cos, self.sin)
                decoder_ops.append_from(keys, k_rot.view(B, nkv * hd), hd, hd, pos)
            decoder_ops.append_from(values, vcols, self.r_v, self.r_v, pos)
        # the fused op writes its output straight in the tiled activation layout the output projection reads
        tiled_attn = self.wo_out.tiled and self.use_fused_k and B <= 64
        attn = self.decode_core(q[None], keys, values, pos, tiled_rows=tiled_attn)
        tiled_attn = attn.dim() == 2                                          # a core may answer row-major
        a2 = attn if tiled_attn else attn[0].reshape(B, nh * self.out_width)   # [64 | B, nh * out_width]
        if residual is not None:
            h, h_tiled = residual
            return self.wo_out.residual(a2, h, h_tiled, x_tiled=tiled_attn, rows=B)
        if out_partials:
            return self.wo_out(a2, x_tiled=tiled_attn, rows=B, mode="partials")
        return self.wo_out(a2, x_tiled=tiled_attn, rows=B).reshape(*shape[:-1], self.hidden_size)

    def decode_core(self, q4, keys, values, pos, tiled_rows=False):
        """The attention core of a decode step over the caches (new rows already appended): q4 [1, B, nh, hd]
        rotated at pos -> [1, B, nh, out_width] bf16. Fused latent op, naive path, or stock decode over the
        cached rotated K, as the layer is configured. With tiled_rows the fused op answers in the tiled
        activation layout, [64, nh * out_width]; the other cores answer row-major regardless."""
        det = bool(self.palu.runtime.deterministic)
        if self.use_fused_k:
            grouped = self.gs > 1
            return fused.palu_sdpa_decode(q4, keys, self.w_rot, self.cs_tab, values,
                                          self.head_dim if grouped else self.r_v, pos,
                                          u_v=self.u_v[None] if grouped else None, scale=self.scale,
                                          out_dtype=torch.bfloat16, group_ranks=self.group_ranks,
                                          tiled_rows=tiled_rows, deterministic=det)
        if self.recon_k:
            return self._naive_attention(q4, keys, values, pos)
        return fused.flash_decode(q4, keys, values, pos, scale=self.scale, head_dim_v=self.r_v, deterministic=det)

    def _recon_len(self) -> int:
        """Positions the naive path rebuilds: PaluRuntime.recon_len (the caller's bound on current_pos + 1)
        rounded up to a multiple of 64, or the whole cache (reference attention.py:518-530)."""
        S = self.palu.runtime.recon_len or self.max_seq_len
        return min(-(-int(S) // 64) * 64, self.max_seq_len)

    def _cache_rows(self, cache, S):
        """[B, G, S, w] row-major bf16 view of the first S positions of a cache (tiled caches converted)."""
        if isinstance(cache, GroupedLatentCache):
            return cache.to_rows()[:, :, :S]
        if isinstance(cache, LatentCache):
            nb = -(-S // 32)
            return LatentCache(cache.data[:, :, :nb], cache.role).to_rows()[:, :, :S]
        return cache[:, :, :S]

    def _naive_attention(self, q4, keys, values, pos):
        """The reference's non-fused decode (attention.py:657-710) on the GPU: K = latent @ u_k for the
        first recon_len positions (bf16 GEMM, fp32 accumulate), Meta RoPE at positions 0..S-1 (the HIP
        rope kernel), grouped V rebuilt per head with u_v, then the stock flash-decode (the MLA op:
        V of width r_v for per-head latents, 128 for grouped ones). Returns [1, B, nh, out_width]."""
        S = self._recon_len()
        if self.palu.runtime.check:
            top = int(pos.max())
            assert top < S, f"recon_len {S} does not cover current_pos max {top}"
        B, nkv, hd, gs = self.max_batch_size, self.n_kv_heads, self.head_dim, self.gs
        per_head = lambda lat: lat if gs == 1 else lat.repeat_interleave(gs, dim=1)     # group -> head latents
        k_lat = per_head(self._cache_rows(keys, S)).contiguous()                          # [B, nkv, S, r_k]
        k = torch.matmul(k_lat, self.u_k.contiguous())                                    # [B, nkv, S, hd] bf16
        rows = B * nkv * S
        rpos = self._naive_pos.get(rows)
        if rpos is None:
            rpos = torch.arange(S, dtype=torch.int32, device=self.device).repeat(B * nkv)
            self._naive_pos[rows] = rpos
        k_rot = decoder_ops.rope_rows(k.view(rows, hd), 1, rpos, self.cos, self.sin).view(B, nkv, S, hd)
        v_lat = self._cache_rows(values, S)
        if gs > 1:
            v = torch.matmul(per_head(v_lat).contiguous(), self.u_v.contiguous())          # [B, nkv, S, hd]
        else:
            v = v_lat.contiguous()                                                         # absorbed V: [B, nkv, S, r_v]
        if v.shape[-1] % 32:   # V widths in 16s exist only as tiled caches (16-wide V tiles): hand both over tiled
            k_rot, v = LatentCache.from_rows(k_rot, "k"), LatentCache.from_rows(v, "v")
        return fused.flash_decode(q4, k_rot, v, pos, scale=self.scale, head_dim_v=self.out_width,
                                  deterministic=bool(self.palu.runtime.deterministic))

    def forward_prefill(self, x, rot_mats=None, user_id=0, page_table=None, chunk_page_table=None,
                        chunk_start_idx=None, kv_cache=None):
        """Prefill of one user (x [1, S, dim] or [1, 1, S, dim], cache row user_id) or of U users at once
        (x [U, S, dim], cache rows user_id .. user_id + U - 1), positions 0 .. S-1."""
        assert page_table is None and chunk_start_idx is None and kv_cache is None
        shape = x.shape
        x3 = x.reshape(-1, shape[-2], self.hidden_size).to(torch.bfloat16)          # [U, S, dim]
        U, S = x3.shape[0], x3.shape[1]
        assert 0 < S <= self.max_seq_len and user_id + U <= self.max_batch_size
        outs = []
        for u in range(U):
            outs.append(self._prefill_one(x3[u], user_id + u))
        return torch.stack(outs).reshape(*shape[:-1], self.hidden_size)

    def _prefill_one(self, x2, user):
        S = x2.shape[0]
        q_pre, k_lat, v_lat = self._split(F.linear(x2, self.wqkv.plain()))   # [S, nh, hd], [S, G, kw], [S, G, r_v]
        pos = torch.arange(S, device=self.device)
        rep_g = lambda t: t.repeat_interleave(self.gs, dim=1)                       # group latent per head
        K = torch.einsum("sgr,grd->sgd", rep_g(k_lat).float(), self.u_k.float()) if self.recon_k else k_lat.float()
        V = torch.einsum("sgr,grd->sgd", rep_g(v_lat).float(), self.u_v.float()) if self.recon_v else v_lat.float()
        q = self._rope(q_pre.float(), pos)
        K = self._rope(K, pos)
        keys, values = self.layer_past
        self._fill(keys, k_lat if self.recon_k else K, user)
        self._fill(values, v_lat, user)
        rep = self.n_heads // self.n_kv_heads
        qh = q.transpose(0, 1)[None]                                                # [1, nh, S, hd] fp32
        Kh = K.repeat_interleave(rep, dim=1).transpose(0, 1)[None].contiguous()
        Vh = V.repeat_interleave(rep, dim=1).transpose(0, 1)[None].contiguous()
        attn = F.scaled_dot_product_attention(qh, Kh, Vh, is_causal=True, scale=self.scale)
        attn = attn[0].transpose(0, 1).reshape(S, self.n_heads * self.head_dim).to(torch.bfloat16)
        return F.linear(attn, self.wo)

    def _fill(self, cache, rows, user_id):
        """Rows [S, G, w] into cache row user_id at positions 0..S-1 (reference ttnn.fill_cache)."""
        r = rows.to(torch.bfloat16).transpose(0, 1)                       # [G, S, w]
        if isinstance(cache, (LatentCache, GroupedLatentCache)):
            cache.write_rows(user_id, 0, r)
        else:
            cache[user_id, :, :r.shape[1]] = r

    def forward(self, x, current_pos=None, rot_mats=None, user_id=0, mode="decode", page_table=None,
                chunk_page_table=None, chunk_start_idx=None, kv_cache=None):
        if str(mode).lower().endswith("prefill"):
            return self.forward_prefill(x, rot_mats, user_id, page_table=page_table, chunk_page_table=chunk_page_table,
                                        chunk_start_idx=chunk_start_idx, kv_cache=kv_cache)
        return self.forward_decode(x, current_pos, rot_mats, page_table=page_table, kv_cache=kv_cache)
