"""Palu low-rank factors -> the tensors the decode path uses (weight layout of the reference's
palu_tt/convert.py, M-LRD and G-LRD).

On-disk format read by ``load_palu_dir`` (convert.py:148-199 of the reference): config.json with
``head_wise_ranks[model.layers.{i}.self_attn.{k,v}_proj]`` = one rank per head group, and in any
*.safetensors file of the directory ``{proj}.VT.weight`` [sum of group ranks, hidden] (the groups'
VT stacked) and ``{proj}.U.{g}.weight`` [group_size * head_dim, r_g]. Group size 1 is M-LRD.

``palu_layer_tensors`` (reference convert.py:227-288) produces the per-layer decode tensors:
  wk_lat_pad / wv_lat_pad [n_kv*hd, hidden]: rows of the fused QKV weight that emit the latents
  u_k [n_kv, r_k, hd]  (Meta head order: reverse_permute of the HF-order factor, transposed)
  u_v [n_kv, r_v, hd]  (identity on the full-rank "fast V" path)
  wo_fused [hidden, n_q*hd]: wo with V's up-projection folded in per query head (M-LRD only)
  w_rot [n_kv, r_k, 2*hd] = [u_k | u_k T]
State-dict keys are ``layers.{i}.attention.palu.{name}`` (reference convert.py:305-306).
"""
import hashlib
import json
import math
import re
from dataclasses import dataclass, field
from pathlib import Path
from typing import Dict, List, Optional

import torch
from safetensors import safe_open

from palu_tt import fused, hf

# Version of the tensor layout produced here; part of every derived cache key.
CONVERT_VERSION = 4


def reverse_permute(t: torch.Tensor, n_heads: int, dim1: int, dim2: int) -> torch.Tensor:
    """HF head-row order -> Meta (interleaved) order: per head, row 2i <- row i and row 2i+1 <- row
    i + hd/2, which turns HF's rotate_half pairing (i, i + hd/2) into adjacent pairs (2i, 2i+1)."""
    half = dim1 // n_heads // 2
    heads = t.reshape(n_heads, 2, half, dim2)
    return torch.stack((heads[:, 0], heads[:, 1]), dim=2).reshape(dim1, dim2)


@dataclass
class PaluRuntime:
    """Decode-path switches of the reference (convert.py:26-58). On MI355X the fused op always runs its
    one schedule; use_fused_k selects it over the naive rebuild, the rest is accepted and recorded."""
    recon_len: Optional[int] = None
    check: bool = False
    use_fused_k: bool = False
    cs_recurrence: bool = False
    fused_k_chunk: Optional[int] = None
    group_heads_per_core: Optional[int] = None
    rot_mode: str = "dst"
    table_mcast: bool = True
    latent_quant_in_prefill: bool = True


@dataclass
class PaluConfig:
    rank_k: List[int]
    rank_v: List[int]
    cache_id: str
    runtime: PaluRuntime = field(default_factory=PaluRuntime)
    latent_dtype: Optional[object] = None
    k_latent_dtype: Optional[object] = None
    v_latent_dtype: Optional[object] = None
    group_size: int = 1
    latent_scale: str = "balanced"
    device_tables: dict = field(default_factory=dict, repr=False, compare=False)


@dataclass
class LowRank:
    """Per-head factors W_h ~= U_h @ VT_h: k_VT [n_kv, r, hidden], k_U [n_kv, hd, r], same for v. With
    group_size > 1 every head of a group carries the group's VT and its own hd-row slice of the group U."""
    k_VT: torch.Tensor
    k_U: torch.Tensor
    v_VT: torch.Tensor
    v_U: torch.Tensor
    group_size: int = 1

    @property
    def r_k(self) -> int:
        return self.k_VT.shape[1]

    @property
    def r_v(self) -> int:
        return self.v_VT.shape[1]


def unit_scale_lowrank(lr: LowRank) -> LowRank:
    """Give every latent component unit scale: column j of the group's U times c_j = ||U[:, j]|| over the
    group's rows, row j of VT divided by c_j. U @ VT is unchanged; zero (padding) columns stay as they are."""
    def rescale(VT, U, gs):
        VT2, U2 = VT.clone(), U.clone()
        for g0 in range(0, U.shape[0], gs):
            heads = slice(g0, g0 + gs)
            c = U[heads].pow(2).sum(dim=(0, 1)).sqrt()
            c = torch.where(c > 0, c, torch.ones_like(c))
            U2[heads] = U[heads] * c
            VT2[heads] = VT[heads] / c[:, None]
        return VT2, U2
    k_VT, k_U = rescale(lr.k_VT, lr.k_U, lr.group_size)
    v_VT, v_U = rescale(lr.v_VT, lr.v_U, lr.group_size)
    return LowRank(k_VT, k_U, v_VT, v_U, group_size=lr.group_size)


def identity_lowrank(hf_attn: Dict[str, torch.Tensor], n_kv_heads: int, head_dim: int) -> LowRank:
    """r == head_dim, VT = the head's weight rows, U = I: the Palu path then computes stock attention."""
    eye = torch.eye(head_dim).expand(n_kv_heads, head_dim, head_dim).contiguous()
    heads = lambda w: w.float().reshape(n_kv_heads, head_dim, -1).contiguous()
    return LowRank(heads(hf_attn["k"]), eye.clone(), heads(hf_attn["v"]), eye.clone())


def _read_palu_layer(tensors, ranks, layer, proj, n_kv_heads, head_dim, rank_multiple):
    """One projection of one layer -> (VT [n_kv, r_pad, hidden], U [n_kv, hd, r_pad], group size)."""
    key = f"model.layers.{layer}.self_attn.{proj}"
    r_list = [int(r) for r in ranks[key]]
    n_groups = len(r_list)
    assert n_kv_heads % n_groups == 0, f"{key}: {n_groups} groups do not divide {n_kv_heads} KV heads"
    gs = n_kv_heads // n_groups
    r_pad = int(math.ceil(max(r_list) / rank_multiple) * rank_multiple)
    VT_all = tensors[f"{key}.VT.weight"]
    VT = torch.zeros(n_kv_heads, r_pad, VT_all.shape[1])
    U = torch.zeros(n_kv_heads, head_dim, r_pad)
    offsets = [0] + list(torch.tensor(r_list).cumsum(0).tolist())
    for g, r in enumerate(r_list):
        U_g = tensors[f"{key}.U.{g}.weight"]
        assert tuple(U_g.shape) == (gs * head_dim, r), f"{key}.U.{g}: {tuple(U_g.shape)} != {(gs * head_dim, r)}"
        heads = slice(g * gs, (g + 1) * gs)
        VT[heads, :r] = VT_all[offsets[g]:offsets[g] + r]
        U[heads, :, :r] = U_g.reshape(gs, head_dim, r)
    return VT, U, gs


def load_palu_dir(palu_dir: Path, n_layers: int, n_kv_heads: int, head_dim: int, rank_multiple: int = 32,
                  latent_scale: str = "balanced") -> Dict[int, LowRank]:
    """Factors of every layer, group ranks zero-padded to the layer's max rounded up to rank_multiple."""
    assert latent_scale in ("balanced", "unit"), f"latent_scale must be 'balanced' or 'unit', got {latent_scale!r}"
    palu_dir = Path(palu_dir)
    ranks = json.loads((palu_dir / "config.json").read_text())["head_wise_ranks"]
    tensors = {}
    for f in sorted(palu_dir.glob("*.safetensors")):
        with safe_open(str(f), framework="pt") as sf:
            for k in sf.keys():
                if ".k_proj." in k or ".v_proj." in k:
                    tensors[k] = sf.get_tensor(k).float()
    out = {}
    for i in range(n_layers):
        k_VT, k_U, gs_k = _read_palu_layer(tensors, ranks, i, "k_proj", n_kv_heads, head_dim, rank_multiple)
        v_VT, v_U, gs_v = _read_palu_layer(tensors, ranks, i, "v_proj", n_kv_heads, head_dim, rank_multiple)
        assert gs_k == gs_v, f"layer {i}: K group size {gs_k} != V group size {gs_v}"
        lr = LowRank(k_VT, k_U, v_VT, v_U, group_size=gs_k)
        out[i] = unit_scale_lowrank(lr) if latent_scale == "unit" else lr
    return out


def palu_dir_cache_id(palu_dir: Path) -> str:
    """Directory name + 8 hex digits of a hash of config.json and every shard's name/size/mtime."""
    palu_dir = Path(palu_dir)
    h = hashlib.sha256((palu_dir / "config.json").read_bytes())
    for f in sorted(palu_dir.glob("*.safetensors")):
        st = f.stat()
        h.update(f"{f.name}:{st.st_size}:{st.st_mtime_ns}\n".encode())
    return f"{re.sub(r'[^A-Za-z0-9._-]', '_', palu_dir.resolve().name)}-{h.hexdigest()[:8]}"


def palu_cache_id_for(palu_dir: Path, latent_scale: str) -> str:
    base = palu_dir_cache_id(palu_dir)
    return base if latent_scale == "balanced" else f"{base}-{latent_scale}"


def palu_layer_tensors(hf_attn: Dict[str, torch.Tensor], lr: LowRank, n_heads: int, n_kv_heads: int,
                       head_dim: int) -> Dict[str, torch.Tensor]:
    """Decode tensors of one layer. Full-rank per-head factors collapse to the stock paths: r_k == hd
    puts reverse_permute(U_k VT_k) (the factorised K weight, Meta order) in the K rows so K needs no
    rebuild; r_v == hd puts U_v VT_v in the V rows and hands an identity u_v downstream ("fast V")."""
    hidden = hf_attn["q"].shape[1]
    r_k, r_v, gs = lr.r_k, lr.r_v, lr.group_size
    hd = head_dim
    dev = lr.k_VT.device
    wk_lat_pad = torch.zeros(n_kv_heads * hd, hidden, device=dev)
    wv_lat_pad = torch.zeros(n_kv_heads * hd, hidden, device=dev)
    fast_v = gs == 1 and r_v == hd
    u_v_eff = torch.eye(hd, device=dev).expand(n_kv_heads, hd, hd) if fast_v else lr.v_U     # [n_kv, hd, r_v]
    for h in range(n_kv_heads):
        g, hh = divmod(h, gs)
        slot = slice(g * gs * hd, g * gs * hd + r_k)
        if gs == 1 and r_k == hd:
            wk_lat_pad[h * hd:(h + 1) * hd] = reverse_permute(lr.k_U[h] @ lr.k_VT[h], 1, hd, hidden)
        elif hh == 0:
            wk_lat_pad[slot] = lr.k_VT[h]
        if fast_v:
            wv_lat_pad[h * hd:(h + 1) * hd] = lr.v_U[h] @ lr.v_VT[h]
        elif hh == 0:
            wv_lat_pad[g * gs * hd:g * gs * hd + r_v] = lr.v_VT[h]
    u_k = torch.stack([reverse_permute(lr.k_U[h], 1, hd, r_k).T for h in range(n_kv_heads)])
    u_v = u_v_eff.transpose(1, 2).contiguous()
    wo = hf_attn["o"].float()
    if gs > 1:
        wo_fused = wo.clone()
    else:
        rep = n_heads // n_kv_heads
        wo_heads = wo.reshape(wo.shape[0], n_heads, hd)                       # [hidden, n_q, hd]
        folded = torch.einsum("oqd,qdr->oqr", wo_heads, u_v_eff.repeat_interleave(rep, dim=0))
        wo_fused = torch.zeros(wo.shape[0], n_heads, hd, device=dev)
        wo_fused[:, :, :r_v] = folded
        wo_fused = wo_fused.reshape(wo.shape[0], n_heads * hd)
    return {"wk_lat_pad": wk_lat_pad, "wv_lat_pad": wv_lat_pad, "u_k": u_k.contiguous(), "u_v": u_v,
            "wo_fused": wo_fused, "w_rot": fused.w_rot_from_u_k(u_k.contiguous())}


def hf_attn_weights(hf_dir: Path, layer: int) -> Dict[str, torch.Tensor]:
    p = f"model.layers.{layer}.self_attn."
    t = hf.load_tensors(hf_dir, lambda k: k.startswith(p) and k.endswith("proj.weight"))
    return {"q": t[p + "q_proj.weight"], "k": t[p + "k_proj.weight"], "v": t[p + "v_proj.weight"],
            "o": t[p + "o_proj.weight"]}


def add_palu_to_state_dict(state_dict: dict, hf_dir: Path, palu_dir: Optional[Path], n_layers: int, n_heads: int,
                           n_kv_heads: int, head_dim: int, latent_scale: str = "balanced") -> PaluConfig:
    """Adds layers.{i}.attention.palu.* for every layer; palu_dir None = identity factors (stock model)."""
    lrs = None if palu_dir is None else load_palu_dir(palu_dir, n_layers, n_kv_heads, head_dim,
                                                       latent_scale=latent_scale)
    rank_k, rank_v = [], []
    for i in range(n_layers):
        w = hf_attn_weights(hf_dir, i)
        lr = identity_lowrank(w, n_kv_heads, head_dim) if lrs is None else lrs[i]
        for name, t in palu_layer_tensors(w, lr, n_heads, n_kv_heads, head_dim).items():
            state_dict[f"layers.{i}.attention.palu.{name}"] = t
        rank_k.append(lr.r_k)
        rank_v.append(lr.r_v)
    cache_id = "identity" if palu_dir is None else palu_cache_id_for(palu_dir, latent_scale)
    sizes = {lr.group_size for lr in lrs.values()} if lrs else {1}
    assert len(sizes) == 1, f"mixed group sizes across layers: {sizes}"
    return PaluConfig(rank_k=rank_k, rank_v=rank_v, cache_id=cache_id, group_size=sizes.pop(),
                      latent_scale=latent_scale)
