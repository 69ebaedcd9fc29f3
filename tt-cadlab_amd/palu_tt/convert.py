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
from dataclasses import dataclass, field
from pathlib import Path
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F
from safetensors import safe_open
from safetensors.torch import save_file

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
    """Decode-path switches of the reference (convert.py:26-58), same fields and defaults. use_fused_k
    selects the fused latent decode over the naive path (K rebuilt and rotated for the first recon_len
    positions, then the stock flash-decode; reference attention.py:657-710); check makes the naive path
    verify that recon_len covers every row's position. The Tensix work-split switches (cs_recurrence,
    fused_k_chunk, group_heads_per_core, rot_mode, table_mcast) and latent_quant_in_prefill are accepted
    and recorded: the MI355X kernels have one schedule and bf16 caches. deterministic (no counterpart in the
    reference, whose op always sums in one order) fixes which wave of a decode workgroup sums which
    32-position block, so repeated decodes are bit-identical; the default hands blocks out from a counter
    (faster where rows differ in length; results differ between calls at the bf16 rounding of the
    softmax probabilities)."""
    recon_len: Optional[int] = None
    check: bool = False
    use_fused_k: bool = False
    cs_recurrence: bool = False
    fused_k_chunk: Optional[int] = None
    group_heads_per_core: Optional[int] = None
    rot_mode: str = "dst"
    table_mcast: bool = True
    latent_quant_in_prefill: bool = True
    deterministic: bool = False


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
    # Per layer, the latent groups' own ranks (K ranks, V ranks) before the padding to rank_k / rank_v, or
    # None. With grouped latents the fused op then reads only each group's own cache columns.
    group_ranks: Optional[List[Optional[Tuple[List[int], List[int]]]]] = None


@dataclass
class LowRank:
    """Per-head factors W_h ~= U_h @ VT_h: k_VT [n_kv, r, hidden], k_U [n_kv, hd, r], same for v. With
    group_size > 1 every head of a group carries the group's VT and its own hd-row slice of the group U."""
    k_VT: torch.Tensor
    k_U: torch.Tensor
    v_VT: torch.Tensor
    v_U: torch.Tensor
    group_size: int = 1
    group_ranks_k: Optional[List[int]] = None    # each group's rank before padding (load_palu_dir fills them)
    group_ranks_v: Optional[List[int]] = None

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
    return LowRank(k_VT, k_U, v_VT, v_U, group_size=lr.group_size, group_ranks_k=lr.group_ranks_k,
                   group_ranks_v=lr.group_ranks_v)


def identity_lowrank(hf_attn: Dict[str, torch.Tensor], n_kv_heads: int, head_dim: int) -> LowRank:
    """r == head_dim, VT = the head's weight rows, U = I: the Palu path then computes stock attention."""
    eye = torch.eye(head_dim).expand(n_kv_heads, head_dim, head_dim).contiguous()
    heads = lambda w: w.float().reshape(n_kv_heads, head_dim, -1).contiguous()
    return LowRank(heads(hf_attn["k"]), eye.clone(), heads(hf_attn["v"]), eye.clone())


class _FactorDump:
    """A Palu factor directory opened for reading: the group ranks of config.json and a name -> shard
    index built from the safetensors headers alone; tensors are read one at a time when asked for, so a
    multi-GB dump is never held in memory whole."""

    def __init__(self, palu_dir: Path):
        self.dir = Path(palu_dir)
        cfg = json.loads((self.dir / "config.json").read_text())
        if "head_wise_ranks" not in cfg:
            raise ValueError(f"{self.dir / 'config.json'} has no 'head_wise_ranks' entry")
        self.ranks = {name: [int(r) for r in rs] for name, rs in cfg["head_wise_ranks"].items()}
        self.where: Dict[str, Path] = {}
        for shard in sorted(self.dir.glob("*.safetensors")):
            with safe_open(str(shard), framework="pt") as f:
                self.where.update(dict.fromkeys(f.keys(), shard))

    def tensor(self, name: str) -> torch.Tensor:
        if name not in self.where:
            raise KeyError(f"{self.dir}: no tensor {name!r} in any *.safetensors shard")
        with safe_open(str(self.where[name]), framework="pt") as f:
            return f.get_tensor(name).float()

    def projection(self, layer: int, proj: str, n_kv_heads: int, head_dim: int, rank_multiple: int):
        """(VT [n_kv, r_pad, hidden], U [n_kv, hd, r_pad], group size, group ranks) of one projection. The stacked VT
        is cut at the group ranks; every group is zero-padded to r_pad (the widest group rounded up to
        rank_multiple) and handed to each of its heads, the head taking its hd rows of the group U."""
        name = f"model.layers.{layer}.self_attn.{proj}"
        if name not in self.ranks:
            raise KeyError(f"{self.dir / 'config.json'}: head_wise_ranks has no entry for {name}")
        group_ranks = self.ranks[name]
        n_groups = len(group_ranks)
        if n_groups == 0 or n_kv_heads % n_groups:
            raise ValueError(f"{name}: {n_groups} rank groups do not divide {n_kv_heads} KV heads")
        gs = n_kv_heads // n_groups
        r_pad = -(-max(group_ranks) // rank_multiple) * rank_multiple
        vt_groups = torch.split(self.tensor(f"{name}.VT.weight"), group_ranks, dim=0)
        u_groups = [self.tensor(f"{name}.U.{g}.weight") for g in range(n_groups)]
        for g, (u, r) in enumerate(zip(u_groups, group_ranks)):
            if tuple(u.shape) != (gs * head_dim, r):
                raise ValueError(f"{name}.U.{g}.weight is {tuple(u.shape)}, expected {(gs * head_dim, r)} "
                                 f"(group of {gs} heads of width {head_dim}, rank {r})")
        VT = torch.stack([F.pad(vt, (0, 0, 0, r_pad - vt.shape[0])) for vt in vt_groups])       # [G, r_pad, hidden]
        U = torch.cat([F.pad(u, (0, r_pad - u.shape[1])).view(gs, head_dim, r_pad) for u in u_groups])
        return VT.repeat_interleave(gs, dim=0).contiguous(), U.contiguous(), gs, list(group_ranks)


def load_palu_dir(palu_dir: Path, n_layers: int, n_kv_heads: int, head_dim: int, rank_multiple: int = 32,
                  latent_scale: str = "balanced") -> Dict[int, LowRank]:
    """Per-layer factors of a Palu dump (a factors-only file or a full dump with the same key names),
    group ranks zero-padded to the layer's widest group rounded up to rank_multiple (no change to any
    product U @ VT). latent_scale "unit" rescales each latent component to unit scale
    (unit_scale_lowrank); "balanced" keeps the dump's split."""
    if latent_scale not in ("balanced", "unit"):
        raise ValueError(f"latent_scale must be 'balanced' or 'unit', got {latent_scale!r}")
    dump = _FactorDump(palu_dir)
    layers = {}
    for i in range(n_layers):
        k_VT, k_U, gs, rk = dump.projection(i, "k_proj", n_kv_heads, head_dim, rank_multiple)
        v_VT, v_U, gs_v, rv = dump.projection(i, "v_proj", n_kv_heads, head_dim, rank_multiple)
        if gs != gs_v:
            raise ValueError(f"layer {i}: k_proj groups {gs} heads and v_proj {gs_v}; the group size must match")
        lr = LowRank(k_VT, k_U, v_VT, v_U, group_size=gs, group_ranks_k=rk, group_ranks_v=rv)
        layers[i] = unit_scale_lowrank(lr) if latent_scale == "unit" else lr
    return layers


def save_palu_dir(palu_dir: Path, layers: Dict[int, Dict[str, List[Tuple[torch.Tensor, torch.Tensor]]]],
                  meta: Optional[dict] = None, shard: str = "palu_lowrank.safetensors") -> Path:
    """Writes the on-disk format load_palu_dir reads. layers[i][proj] (proj "k_proj" / "v_proj") is the
    list of per-group factors (U_g [group_size * hd, r_g], VT_g [r_g, hidden]); the group VTs are stacked
    into one {proj}.VT.weight and config.json["head_wise_ranks"] records r_g per group."""
    palu_dir = Path(palu_dir)
    palu_dir.mkdir(parents=True, exist_ok=True)
    tensors, ranks = {}, {}
    for i, projs in sorted(layers.items()):
        for proj, groups in projs.items():
            name = f"model.layers.{i}.self_attn.{proj}"
            ranks[name] = [int(vt.shape[0]) for _, vt in groups]
            tensors[f"{name}.VT.weight"] = torch.cat([vt.float() for _, vt in groups]).contiguous()
            tensors.update({f"{name}.U.{g}.weight": u.float().contiguous() for g, (u, _) in enumerate(groups)})
    save_file(tensors, str(palu_dir / shard))
    (palu_dir / "config.json").write_text(json.dumps({"head_wise_ranks": ranks, **(meta or {})}, indent=1))
    return palu_dir


def _sampled_digest(path: Path, windows: int = 16, width: int = 4096) -> bytes:
    """sha256 of a safetensors shard's header plus `windows` evenly spaced `width`-byte windows of its data:
    a content fingerprint that reads a few tens of KB however large the shard is."""
    h = hashlib.sha256()
    size = path.stat().st_size
    with open(path, "rb") as f:
        n = int.from_bytes(f.read(8), "little")
        h.update(f.read(n))
        lo = 8 + n
        span = max(size - lo - width, 0)
        for w in range(windows):
            f.seek(lo + (span * w) // max(windows - 1, 1))
            h.update(f.read(width))
    h.update(str(size).encode())
    return h.digest()


def palu_dir_cache_id(palu_dir: Path) -> str:
    """Id of a dump's weight set: the directory name (filesystem-safe) and 8 hex digits of a fingerprint
    of config.json's bytes and every shard's header and sampled contents, so it changes when the ranks or
    the tensors change and not when files are merely touched."""
    palu_dir = Path(palu_dir)
    h = hashlib.sha256((palu_dir / "config.json").read_bytes())
    for shard in sorted(palu_dir.glob("*.safetensors")):
        h.update(shard.name.encode() + b"\0" + _sampled_digest(shard))
    safe_name = "".join(c if (c.isalnum() or c in "._-") else "_" for c in palu_dir.resolve().name)
    return f"{safe_name}-{h.hexdigest()[:8]}"


def palu_cache_id_for(palu_dir: Path, latent_scale: str) -> str:
    """The id under a latent scale: rescaled factors share shapes and dtypes with the balanced ones, so a
    cache keyed by them must tell the two apart ("-unit" suffix)."""
    return palu_dir_cache_id(palu_dir) + ("" if latent_scale == "balanced" else f"-{latent_scale}")


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


_ATTN_PROJ = {"q": "q_proj", "k": "k_proj", "v": "v_proj", "o": "o_proj"}


def hf_attn_weights(hf_dir: Path, layer: int) -> Dict[str, torch.Tensor]:
    """The four attention projection weights of one layer of an HF checkpoint, keyed q / k / v / o."""
    names = {f"model.layers.{layer}.self_attn.{full}.weight": short for short, full in _ATTN_PROJ.items()}
    found = hf.load_tensors(hf_dir, names.__contains__)
    missing = sorted(set(names) - set(found))
    if missing:
        raise KeyError(f"{hf_dir}: missing {missing}")
    return {names[k]: t for k, t in found.items()}


def add_palu_to_state_dict(state_dict: dict, hf_dir: Path, palu_dir: Optional[Path], n_layers: int, n_heads: int,
                           n_kv_heads: int, head_dim: int, latent_scale: str = "balanced") -> PaluConfig:
    """Puts layers.{i}.attention.palu.{wk_lat_pad, wv_lat_pad, u_k, u_v, wo_fused, w_rot} into state_dict
    for every layer and returns the PaluConfig describing them. palu_dir None runs the stock model through
    the Palu path (identity factors, cache id "identity")."""
    factors = (load_palu_dir(palu_dir, n_layers, n_kv_heads, head_dim, latent_scale=latent_scale)
               if palu_dir is not None else None)
    group_sizes = set()
    per_layer_ranks, group_ranks = [], []
    for i in range(n_layers):
        attn = hf_attn_weights(hf_dir, i)
        lr = factors[i] if factors is not None else identity_lowrank(attn, n_kv_heads, head_dim)
        tensors = palu_layer_tensors(attn, lr, n_heads, n_kv_heads, head_dim)
        state_dict.update({f"layers.{i}.attention.palu.{k}": t for k, t in tensors.items()})
        per_layer_ranks.append((lr.r_k, lr.r_v))
        group_ranks.append(None if lr.group_ranks_k is None else (lr.group_ranks_k, lr.group_ranks_v))
        group_sizes.add(lr.group_size)
    if len(group_sizes) > 1:
        raise ValueError(f"layers use different group sizes {sorted(group_sizes)}; one model has one group size")
    return PaluConfig(rank_k=[rk for rk, _ in per_layer_ranks], rank_v=[rv for _, rv in per_layer_ranks],
                      cache_id="identity" if palu_dir is None else palu_cache_id_for(palu_dir, latent_scale),
                      group_size=group_sizes.pop() if group_sizes else 1, latent_scale=latent_scale,
                      group_ranks=group_ranks if factors is not None else None)
