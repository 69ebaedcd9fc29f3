"""CPU fp32 oracle for Palu's fused latent flash-decode. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import this module, and only
as the oracle that results are compared with (or, in bench.py, as the CPU path timed beside the GPU). The product
(tt-cadlab_amd/palu_tt) never imports it and fails loudly when its HIP library is missing.

Everything here is a restatement, written from the mathematics the reference implements, of:

* palu_tt/fused.py:36-107  -- pair-rotation matrix T, [u_k | u_k T], chunk rule, Meta-interleaved
  cos/sin tables, [cos | sin] table, Phase 2 step row, and ``reference_decode`` (the fp32 model of
  ttnn.transformer.palu_sdpa_decode);
* palu_tt/reference.py:14-92 -- ``PaluRefAttention`` (HF conventions: rotate_half RoPE on unpermuted
  heads, latent caches, full K/V rebuild, GQA, causal softmax, o_proj), ``LowRankProj`` and the
  low-rank Llama (``lowrank_llama``, on transformers' LlamaForCausalLM);
* palu_tt/compress.py:12-23  -- per-head truncated SVD with Palu's balanced split;
* tt-metal load_checkpoints.reverse_permute (HF head order -> Meta interleaved order), as the
  reference's audit restates it (docs/audit/reports/scripts/math_check.py:10-11);
* the llama3 rope-frequency scaling (Meta's published formula, as transformers'
  modeling_rope_utils._compute_llama3_parameters and tt_transformers' rope.apply_scaling compute it).

How each function is pinned (tests/test_oracle.py):
  rope_transformation_matrix  -- pair-rotation property (ref tests/test_fused.py:8-16)
  inv_freq / cos_sin_tables   -- bit-compared with transformers' LlamaRotaryEmbedding (llama3 scaling)
                                 after the HF -> Meta column rearrangement; cos[0] == 1; interleave
  chunk_size                  -- known answers of ref tests/test_fused.py:28-30
  reference_decode            -- brute-force per-(b, h) softmax loop (ref tests/test_fused.py:76-89);
                                 rotation == RoPE on rebuilt K (92-103); u_v mode == prebuilt V
                                 (106-115); and equality with PaluRefAttention through the converter
  PaluRefAttention            -- identity factors == transformers LlamaAttention; prefill-then-decode
                                 == fresh prefill (ref tests/test_reference.py:17-35)
  reverse_permute             -- equals the Meta interleave of HF's rotate_half halves
  svd_per_head                -- exact at full rank, error monotone in rank (ref tests/test_compress.py)
  gather_pages                -- element-by-element position -> (page, row) loop
  LowRankProj / lowrank_llama -- LowRankProj == the dense U @ VT projection; at full-rank factors the
                                 model equals transformers' dense LlamaForCausalLM on the same weights,
                                 and its last-layer attention equals PaluRefAttention on the same input
"""
import math
from dataclasses import dataclass
from typing import Optional

import torch

MAX_CHUNK = 512


# ------------------------------------------------------------------------------------------------
# RoPE pieces (palu_tt/fused.py:36-79)

def rope_transformation_matrix(head_dim: int) -> torch.Tensor:
    """[hd, hd] with x @ T = (-x1, x0) on every adjacent pair (T[2i, 2i+1] = 1, T[2i+1, 2i] = -1)."""
    T = torch.zeros(head_dim, head_dim)
    for i in range(0, head_dim, 2):
        T[i, i + 1] = 1.0
        T[i + 1, i] = -1.0
    return T


def w_rot_from_u_k(u_k: torch.Tensor) -> torch.Tensor:
    return torch.cat([u_k, u_k @ rope_transformation_matrix(u_k.shape[-1])], dim=-1)


def chunk_size(seq_len: int) -> int:
    """Largest power of two dividing seq_len, capped at 512 (palu_tt/fused.py:54-59)."""
    assert seq_len > 0
    c = 1
    while seq_len % (c * 2) == 0 and c * 2 <= MAX_CHUNK:
        c *= 2
    return c


def _scaling_field(rs, name, default=None):
    if rs is None:
        return default
    if isinstance(rs, dict):
        return rs.get(name, default)
    return getattr(rs, name, default)


def inv_freq(head_dim: int, theta: float, rope_scaling=None) -> torch.Tensor:
    """fp32 RoPE frequencies theta^(-2i/hd), llama3-scaled when rope_scaling carries a factor."""
    exps = torch.arange(0, head_dim, 2).float() / head_dim
    f = 1.0 / (theta ** exps)
    factor = _scaling_field(rope_scaling, "factor")
    if factor is None:
        return f
    low = float(_scaling_field(rope_scaling, "low_freq_factor", 1.0))
    high = float(_scaling_field(rope_scaling, "high_freq_factor", 4.0))
    orig = float(_scaling_field(rope_scaling, "original_max_position_embeddings", 8192))
    long_wavelen = orig / low          # wavelengths above this are slowed by the full factor
    short_wavelen = orig / high        # wavelengths below this are untouched
    out = []
    for fi in f:                       # element by element, in fp32 tensor arithmetic
        wl = 2 * math.pi / fi
        if wl < short_wavelen:
            out.append(fi)
        elif wl > long_wavelen:
            out.append(fi / factor)
        else:
            s = (orig / wl - low) / (high - low)
            out.append((1 - s) * fi / factor + s * fi)
    return torch.stack(out).float()


def cos_sin_tables(head_dim: int, seq_len: int, theta: float, rope_scaling=None):
    """Meta-interleaved fp32 (cos, sin), each [seq_len + 513, head_dim]: column 2i and 2i+1 hold angle
    t * f_i, the angle rounded to fp32 before cos/sin (palu_tt/fused.py:62-68)."""
    n = seq_len + MAX_CHUNK + 1
    f = inv_freq(head_dim, theta, rope_scaling)
    ang = torch.arange(n).float()[:, None] * f[None, :]           # [n, hd/2], one fp32 product each
    cos = ang.cos().repeat_interleave(2, dim=1)
    sin = ang.sin().repeat_interleave(2, dim=1)
    return cos.contiguous(), sin.contiguous()


def cs_table(cos, sin, seq_len):
    return torch.cat([cos[:seq_len], sin[:seq_len]], dim=-1)


def rot_step_table(cos, sin, chunk):
    return torch.cat([cos[chunk], sin[chunk]]).expand(32, -1).contiguous().float()


def meta_rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x * cos + (x @ T) * sin on the last dim (Meta-interleaved pairs), written pairwise."""
    x0, x1 = x[..., 0::2], x[..., 1::2]
    c, s = cos[..., 0::2], sin[..., 0::2]
    out = torch.empty_like(x)
    out[..., 0::2] = x0 * c - x1 * s
    out[..., 1::2] = x1 * c + x0 * s
    return out


# ------------------------------------------------------------------------------------------------
# The op model (palu_tt/fused.py:82-107)

@torch.no_grad()
def reference_decode(q, k_lat, u_k, v_lat, cur_pos, cos, sin, scale: float, u_v=None) -> torch.Tensor:
    """fp32 model of palu_sdpa_decode.

    q [1, B, nh, hd] (already rotated), k_lat [B, n_lat, S, r_k], u_k [nkv, r_k, hd], v_lat [B, n_lat, S,
    r_v], cur_pos [B] (inclusive), cos/sin [>= S, hd] Meta-interleaved. Query head h attends KV head
    h // (nh // nkv); KV head j reads latent head j // (nkv // n_lat) (n_lat == nkv for M-LRD).
    u_v [nkv, r_v, hd] rebuilds V per head; without it the V latent is attended directly (absorbed V).
    Returns [1, B, nh, r_v or hd] fp32. Rows are computed one batch row at a time (same arithmetic
    as materialising every row at once, bounded memory)."""
    B, n_lat, S, _ = k_lat.shape
    nh = q.shape[2]
    nkv = u_k.shape[0]
    rep, hpg = nh // nkv, nkv // n_lat
    u_k = u_k.float()
    u_v = None if u_v is None else u_v.float()
    c, s = cos[:S].float(), sin[:S].float()
    outs = []
    for b in range(B):
        L = int(cur_pos[b]) + 1
        lat_k = k_lat[b].float().repeat_interleave(hpg, dim=0)[:, :L]           # [nkv, L, r_k]
        K = torch.einsum("hsr,hrd->hsd", lat_k, u_k)
        K = meta_rotate(K, c[None, :L], s[None, :L])
        V = v_lat[b].float().repeat_interleave(hpg, dim=0)[:, :L]
        if u_v is not None:
            V = torch.einsum("hsr,hrd->hsd", V, u_v)
        K = K.repeat_interleave(rep, dim=0)                                   # [nh, L, hd]
        V = V.repeat_interleave(rep, dim=0)
        sc = torch.einsum("hd,hsd->hs", q[0, b].float(), K) * scale
        p = torch.softmax(sc, dim=-1)
        outs.append(torch.einsum("hs,hsr->hr", p, V))
    return torch.stack(outs)[None]


def gather_pages(pool: torch.Tensor, page_table: torch.Tensor) -> torch.Tensor:
    """Paged cache -> contiguous rows: pool [n_pages, G, page_size, r], page_table [B, max_pages] ->
    [B, G, max_pages * page_size, r], position p of row b taken from page page_table[b, p // page_size],
    row p % page_size (the paged-cache convention of ttnn's paged decode and paged_update_cache)."""
    pages = pool[page_table.long()]                        # [B, max_pages, G, page_size, r]
    B, mp, G, ps, r = pages.shape
    return pages.permute(0, 2, 1, 3, 4).reshape(B, G, mp * ps, r)


@torch.no_grad()
def full_kv_decode(q, k, v, cur_pos, scale: float) -> torch.Tensor:
    """fp32 stock decode over full rotated K [B, nkv, S, hd] and V [B, nkv, S, dv] -> [1, B, nh, dv]."""
    B, nkv, S, _ = k.shape
    nh = q.shape[2]
    rep = nh // nkv
    outs = []
    for b in range(B):
        L = int(cur_pos[b]) + 1
        K = k[b, :, :L].float().repeat_interleave(rep, dim=0)
        V = v[b, :, :L].float().repeat_interleave(rep, dim=0)
        sc = torch.einsum("hd,hsd->hs", q[0, b].float(), K) * scale
        outs.append(torch.einsum("hs,hsr->hr", torch.softmax(sc, dim=-1), V))
    return torch.stack(outs)[None]


# ------------------------------------------------------------------------------------------------
# Layer oracle on HF conventions (palu_tt/reference.py:14-71)

def reverse_permute(t: torch.Tensor, n_heads: int, dim1: int, dim2: int) -> torch.Tensor:
    """HF head rows [x_0..x_{d/2-1}, y_0..y_{d/2-1}] -> Meta rows [x_0, y_0, x_1, y_1, ...] per head."""
    return t.view(n_heads, 2, dim1 // n_heads // 2, dim2).transpose(1, 2).reshape(dim1, dim2)


def hf_cos_sin(positions: torch.Tensor, head_dim: int, theta: float, rope_scaling=None):
    """HF-layout cos/sin [len, hd] = cat(angles, angles) for the given positions."""
    f = inv_freq(head_dim, theta, rope_scaling)
    ang = positions.float()[:, None] * f[None, :]
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos(), emb.sin()


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


@dataclass
class Factors:
    """Per-head low-rank factors: W_h ~= U_h @ VT_h (k_VT [nkv, r, dim], k_U [nkv, hd, r]; same for v)."""
    k_VT: torch.Tensor
    k_U: torch.Tensor
    v_VT: torch.Tensor
    v_U: torch.Tensor


def identity_factors(wk: torch.Tensor, wv: torch.Tensor, n_kv: int, head_dim: int) -> Factors:
    eye = torch.eye(head_dim).expand(n_kv, head_dim, head_dim).contiguous()
    return Factors(wk.float().reshape(n_kv, head_dim, -1).contiguous(), eye.clone(),
                   wv.float().reshape(n_kv, head_dim, -1).contiguous(), eye.clone())


class PaluRefAttention:
    """fp32 attention layer with latent K/V caches (palu_tt/reference.py:14-55)."""

    def __init__(self, n_heads: int, n_kv: int, head_dim: int, theta: float, rope_scaling, wq, wo, factors: Factors):
        self.nh, self.nkv, self.hd = n_heads, n_kv, head_dim
        self.theta, self.rope_scaling = theta, rope_scaling
        self.wq, self.wo = wq.float(), wo.float()
        self.f = factors
        self.cache_k_lat = None
        self.cache_v_lat = None

    @torch.no_grad()
    def forward(self, x: torch.Tensor, start_pos: int, return_attention: bool = False):
        """Output [B, S, dim]; with return_attention also the attention output before o_proj, softmax(q K^T /
        sqrt(hd)) V per head, [B, S, nh * hd] (heads in order, each head's dims in v_proj's row order)."""
        B, S, _ = x.shape
        q = (x @ self.wq.T).view(B, S, self.nh, self.hd).transpose(1, 2)
        k_lat = torch.einsum("bsd,hrd->bhsr", x, self.f.k_VT)
        v_lat = torch.einsum("bsd,hrd->bhsr", x, self.f.v_VT)
        if self.cache_k_lat is None or start_pos == 0:
            self.cache_k_lat, self.cache_v_lat = k_lat, v_lat
        else:
            assert self.cache_k_lat.shape[2] == start_pos
            self.cache_k_lat = torch.cat([self.cache_k_lat, k_lat], dim=2)
            self.cache_v_lat = torch.cat([self.cache_v_lat, v_lat], dim=2)
        T = self.cache_k_lat.shape[2]
        K = torch.einsum("bhtr,hdr->bhtd", self.cache_k_lat, self.f.k_U)
        V = torch.einsum("bhtr,hdr->bhtd", self.cache_v_lat, self.f.v_U)
        cq, sq = hf_cos_sin(torch.arange(start_pos, start_pos + S), self.hd, self.theta, self.rope_scaling)
        ck, sk = hf_cos_sin(torch.arange(T), self.hd, self.theta, self.rope_scaling)
        q = q * cq + rotate_half(q) * sq
        K = K * ck + rotate_half(K) * sk
        rep = self.nh // self.nkv
        K = K.repeat_interleave(rep, dim=1)
        V = V.repeat_interleave(rep, dim=1)
        scores = q @ K.transpose(-1, -2) / math.sqrt(self.hd)
        mask = torch.ones(S, T, dtype=torch.bool).tril(diagonal=start_pos)
        scores = scores.masked_fill(~mask, float("-inf"))
        out = (torch.softmax(scores, dim=-1) @ V).transpose(1, 2).reshape(B, S, self.nh * self.hd)
        return (out @ self.wo.T, out) if return_attention else out @ self.wo.T


class LowRankProj(torch.nn.Module):
    """x -> concat_h (x @ VT_h^T) @ U_h^T: a k_proj / v_proj drop-in that computes through the latent
    (palu_tt/reference.py:58-71)."""

    def __init__(self, VT: torch.Tensor, U: torch.Tensor):
        super().__init__()
        self.VT = VT.float()                                       # [n, r, dim]
        self.U = U.float()                                         # [n, hd, r]

    def forward(self, x):
        lat = torch.einsum("...d,hrd->...hr", x, self.VT)
        return torch.einsum("...hr,hdr->...hd", lat, self.U).flatten(-2)


def lowrank_llama(cfg: dict, weights: dict, factors):
    """fp32 transformers LlamaForCausalLM whose k_proj / v_proj are LowRankProj(factors[i]) (palu_tt/
    reference.py:74-92, built from given weights instead of a checkpoint directory). cfg: dim, n_layers,
    n_heads, n_kv_heads, head_dim, vocab_size, ffn_dim, norm_eps, rope_theta, rope_scaling. weights: the
    HF state dict minus k_proj / v_proj (q_proj in HF head order)."""
    import transformers
    hf_cfg = transformers.LlamaConfig(
        vocab_size=cfg["vocab_size"], hidden_size=cfg["dim"], intermediate_size=cfg["ffn_dim"],
        num_hidden_layers=cfg["n_layers"], num_attention_heads=cfg["n_heads"], num_key_value_heads=cfg["n_kv_heads"],
        head_dim=cfg["head_dim"], rms_norm_eps=cfg["norm_eps"], rope_theta=cfg["rope_theta"],
        rope_scaling=cfg["rope_scaling"], max_position_embeddings=131072, tie_word_embeddings=False,
        attn_implementation="eager")
    model = transformers.LlamaForCausalLM(hf_cfg).float().eval()
    missing, unexpected = model.load_state_dict({k: v.float() for k, v in weights.items()}, strict=False)
    assert not unexpected and all(k.endswith(("k_proj.weight", "v_proj.weight")) for k in missing), (missing, unexpected)
    for layer, f in zip(model.model.layers, factors):
        layer.self_attn.k_proj = LowRankProj(f.k_VT, f.k_U)
        layer.self_attn.v_proj = LowRankProj(f.v_VT, f.v_U)
    return model


# ------------------------------------------------------------------------------------------------
# Factor production (palu_tt/compress.py:12-23)

def svd_per_head(W: torch.Tensor, n_heads: int, rank: int):
    """W [n*hd, dim] -> U [n, hd, r] = U_r sqrt(S), VT [n, r, dim] = sqrt(S) Vt_r."""
    hd = W.shape[0] // n_heads
    Wh = W.float().reshape(n_heads, hd, -1)
    Us, VTs = [], []
    for h in range(n_heads):
        U, S, Vt = torch.linalg.svd(Wh[h], full_matrices=False)
        r = torch.sqrt(S[:rank])
        Us.append(U[:, :rank] * r[None, :])
        VTs.append(r[:, None] * Vt[:rank])
    return torch.stack(Us), torch.stack(VTs)


# ------------------------------------------------------------------------------------------------
# Comparison metrics used by the parity tests

def pcc(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double().flatten(), b.double().flatten()
    a, b = a - a.mean(), b - b.mean()
    den = a.norm() * b.norm()
    return float((a @ b) / den) if den > 0 else float(torch.equal(a, b))


def cosine(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double().flatten(), b.double().flatten()
    den = a.norm() * b.norm()
    return float((a @ b) / den) if den > 0 else float(torch.equal(a, b))


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.double() - b.double()).abs().max())
