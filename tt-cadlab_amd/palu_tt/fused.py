"""Host side of the fused latent flash-decode: the tables the kernel reads and the op entry points.

Mirrors the reference module palu_tt/fused.py (table builders, fused.py:36-79) and the op it calls,
ttnn.transformer.palu_sdpa_decode (call site palu_tt/attention.py:632-639; interface
docs/superpowers/specs/2026-09-10-palu-tt-stage2-design.md:47-81). The op runs as hand-written HIP on
MI355X through libpalu_mi355x.so; this module only validates, shapes and launches.

Layouts (all torch tensors on the GPU unless noted):
  q        [1, B, n_q, 128] bf16, rotated at its own position
  k_latent [B, n_groups, S, r_k] bf16, v_latent [B, n_groups, S, r_v] bf16
  w_rot    [1, n_kv, r_k, 256] bf16 = [u_k | u_k T]
  cs_tab   [1, 1, >= S, 256] fp32 (or bf16) = [cos | sin], Meta-interleaved
  cur_pos  [B] int32, inclusive last valid position per row
The output is [1, B, n_q, head_dim_v]: head_dim_v == r_v for the absorbed-V path.
Either cache may instead be a ``palu_tt.cache.LatentCache`` (same logical shape, tiled HBM layout, the
fast path); both caches of one call use the same layout.

The reference's Tensix switches (rot_step/trans_mat selecting Phase 2, rot_mode, table_mcast,
heads_per_core, program_config chunk) are accepted and validated with the reference's messages. The
MI355X kernel has one schedule: K rows are rotated by their offset inside a 32-position block from
an LDS-resident table and the query is rotated back by the block base, which is the reference's Phase 2
identity (fused.py:1-24) with a fixed chunk; results do not depend on those switches.
"""
import ctypes
import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from palu_tt import _native, decoder_ops
from palu_tt.cache import GroupedLatentCache, LatentCache

MAX_CHUNK = 512          # the reference's cap on the static K chunk (ttnn sdpa_decode)
HEAD_DIM = 128
ROT_MODES = {"legacy": 0, "pack": 1, "dst": 2}


# ------------------------------------------------------------------------------------------------
# Tables (palu_tt/fused.py:36-79)

def rope_transformation_matrix(head_dim: int) -> torch.Tensor:
    """[hd, hd] pair rotation: x @ T maps every adjacent pair (x0, x1) to (-x1, x0)."""
    idx = torch.arange(0, head_dim, 2)
    T = torch.zeros(head_dim, head_dim)
    T[idx, idx + 1] = 1.0
    T[idx + 1, idx] = -1.0
    return T


def trans_mat_tile() -> torch.Tensor:
    """[1, 1, 32, 32]: the pair rotation on one 32-column tile (reference Phase 2 input)."""
    return rope_transformation_matrix(32)[None, None]


def w_rot_from_u_k(u_k: torch.Tensor) -> torch.Tensor:
    """u_k [n_kv, r_k, hd] -> [n_kv, r_k, 2*hd] = [u_k | u_k @ T]."""
    return torch.cat([u_k, u_k @ rope_transformation_matrix(u_k.shape[-1]).to(u_k)], dim=-1)


def chunk_size(seq_len: int) -> int:
    """Largest power of two dividing seq_len, capped at MAX_CHUNK (the reference's static chunk rule)."""
    assert seq_len > 0, f"chunk_size requires seq_len > 0, got {seq_len}"
    return min(MAX_CHUNK, seq_len & -seq_len)


def _rope_field(rope_scaling, name, default=None):
    if rope_scaling is None:
        return default
    if isinstance(rope_scaling, dict):
        return rope_scaling.get(name, default)
    return getattr(rope_scaling, name, default)


def rope_frequencies(head_dim: int, theta: float, rope_scaling=None) -> torch.Tensor:
    """fp32 [hd/2] RoPE frequencies; llama3 scaling (factor, low/high frequency factors, original
    context) when rope_scaling carries a factor, e.g. Llama-3.1's factor 8, 1, 4, 8192."""
    base = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    factor = _rope_field(rope_scaling, "factor")
    if factor is None:
        return base
    low = float(_rope_field(rope_scaling, "low_freq_factor", 1.0))
    high = float(_rope_field(rope_scaling, "high_freq_factor", 4.0))
    orig = float(_rope_field(rope_scaling, "original_max_position_embeddings", 8192))
    wavelen = 2 * math.pi / base
    slow = torch.where(wavelen > orig / low, base / factor, base)
    smooth = (orig / wavelen - low) / (high - low)
    blended = (1 - smooth) * slow / factor + smooth * slow
    middle = ~(wavelen < orig / high) & ~(wavelen > orig / low)
    return torch.where(middle, blended, slow).float()


def cos_sin_tables(head_dim: int, seq_len: int, theta: float, rope_scaling=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Meta-interleaved fp32 cos, sin, each [seq_len + MAX_CHUNK + 1, head_dim] (the extra rows hold the
    step constants): columns 2i and 2i+1 carry angle fp32(t * f_i)."""
    n = seq_len + MAX_CHUNK + 1
    ang = torch.outer(torch.arange(n, dtype=torch.float32), rope_frequencies(head_dim, theta, rope_scaling))
    return (torch.repeat_interleave(ang.cos(), 2, dim=1).contiguous(),
            torch.repeat_interleave(ang.sin(), 2, dim=1).contiguous())


def cs_table(cos: torch.Tensor, sin: torch.Tensor, seq_len: int) -> torch.Tensor:
    """[seq_len, 2*hd] = [cos | sin] for positions 0..seq_len-1."""
    return torch.cat([cos[:seq_len], sin[:seq_len]], dim=-1)


def rot_step_table(cos: torch.Tensor, sin: torch.Tensor, chunk: int) -> torch.Tensor:
    """[32, 2*hd] fp32: [cos(chunk f) | sin(chunk f)] on every row (the reference's Phase 2 step)."""
    return torch.cat([cos[chunk], sin[chunk]]).expand(32, -1).contiguous().float()


def apply_rope_meta(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x * cos + (x @ T) * sin over the last dim (Meta-interleaved pairs), cos/sin broadcastable to x:
    the rotation the reference applies to q with rotary_embedding_llama before the fused op."""
    x2 = x.float().unflatten(-1, (-1, 2))
    c, s = cos.float()[..., 0::2], sin.float()[..., 0::2]
    y0 = x2[..., 0] * c - x2[..., 1] * s
    y1 = x2[..., 1] * c + x2[..., 0] * s
    return torch.stack((y0, y1), dim=-1).flatten(-2)


# ------------------------------------------------------------------------------------------------
# Program config stand-ins (the reference passes ttnn.SDPAProgramConfig / compute kernel configs)

@dataclass
class SDPAProgramConfig:
    compute_with_storage_grid_size: Tuple[int, int] = (8, 8)
    q_chunk_size: int = 0
    k_chunk_size: int = 0
    exp_approx_mode: bool = False


def _k_chunk(program_config) -> int:
    if program_config is None:
        return 0
    return int(getattr(program_config, "k_chunk_size", 0) or 0)


def _grid_cores(program_config) -> Optional[int]:
    grid = getattr(program_config, "compute_with_storage_grid_size", None) if program_config is not None else None
    if grid is None:
        return None
    gx, gy = (grid.x, grid.y) if hasattr(grid, "x") else tuple(grid)
    return int(gx) * int(gy)


# ------------------------------------------------------------------------------------------------
# Op entry points

_DTYPES = {torch.float32: _native.DTYPE_F32, torch.bfloat16: _native.DTYPE_BF16}


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _as_dev(t: torch.Tensor, name: str, dtype=None, device=None) -> torch.Tensor:
    _require(isinstance(t, torch.Tensor), f"{name} must be a torch.Tensor")
    _require(t.is_cuda, f"{name} must live on the GPU (got {t.device})")
    if device is not None:
        _require(t.device == device, f"{name} is on {t.device}, expected {device}")
    if dtype is not None:
        _require(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")
    _require(t.is_contiguous(), f"{name} must be contiguous")
    return t


def _cache_arg(t, name: str, device, role: Optional[str] = None):
    """(storage tensor, logical shape, layout id) of a row-major tensor or a LatentCache; a tiled cache
    passed where the op reads K (role "k") or V (role "v") must be stored in that role's tile order."""
    if isinstance(t, GroupedLatentCache):
        _as_dev(t.data, name, torch.bfloat16, device)
        _require(role is not None and t.role == role,
                 f"{name} is a GroupedLatentCache in {t.role!r} tile order; this argument reads a {role!r} cache")
        return t.data, tuple(t.shape), _native.LAYOUT_TILED_GROUPED
    if isinstance(t, LatentCache):
        _as_dev(t.data, name, torch.bfloat16, device)
        _require(role is None or t.role == role,
                 f"{name} is a LatentCache in {t.role!r} tile order; this argument reads a {role!r} cache")
        layout = _native.LAYOUT_TILED if t.role == "k" else _native.LAYOUT_TILED_V
        return t.data, tuple(t.shape), (_native.LAYOUT_TILED if role is not None else layout)
    _require(isinstance(t, torch.Tensor) and t.dim() == 4, f"{name} must be [B, n_groups, S, width] or a LatentCache")
    _as_dev(t, name, torch.bfloat16, device)
    return t, tuple(t.shape), _native.LAYOUT_ROWS


def _workspace(batch: int, n_kv: int, seq_len: int, width: int, device, workspace):
    need = _native.load().palu_decode_workspace_bytes(batch, n_kv, seq_len, width)
    if need == 0:
        return None, 0
    if workspace is not None:
        _require(workspace.is_cuda and workspace.numel() * workspace.element_size() >= need,
                 f"workspace must hold {need} bytes on the GPU")
        return workspace, workspace.numel() * workspace.element_size()
    return torch.empty(need, dtype=torch.uint8, device=device), need


def _glrd_workspace(batch: int, n_q: int, n_kv: int, n_groups: int, seq_len: int, r_v: int, device, workspace):
    """Workspace of the grouped-latent path: partial scores and latent PV partials between its passes."""
    need = _native.load().palu_glrd_workspace_bytes(batch, n_q, n_kv, n_groups, seq_len, r_v)
    if workspace is not None:
        _require(workspace.is_cuda and workspace.numel() * workspace.element_size() >= need,
                 f"workspace must hold {need} bytes on the GPU (palu_glrd_workspace_bytes)")
        return workspace, workspace.numel() * workspace.element_size()
    return torch.empty(max(need, 1), dtype=torch.uint8, device=device), need


def _cur_pos(cur_pos_tensor: torch.Tensor, batch: int, device) -> torch.Tensor:
    _require(isinstance(cur_pos_tensor, torch.Tensor), "cur_pos_tensor must be a torch.Tensor")
    cp = cur_pos_tensor.reshape(-1)
    _require(cp.numel() == batch, f"cur_pos_tensor has {cp.numel()} entries for batch {batch}")
    if cp.device != device or cp.dtype != torch.int32:
        cp = cp.to(device=device, dtype=torch.int32)
    return cp.contiguous()


def _page_table(page_table_tensor, batch: int, device) -> torch.Tensor:
    _require(isinstance(page_table_tensor, torch.Tensor) and page_table_tensor.dim() == 2,
             "page_table_tensor must be [B, max_pages_per_seq] int32")
    _require(page_table_tensor.shape[0] == batch,
             f"page_table_tensor has {page_table_tensor.shape[0]} rows for batch {batch}")
    pt = page_table_tensor
    if pt.device != device or pt.dtype != torch.int32:
        pt = pt.to(device=device, dtype=torch.int32)
    return pt.contiguous()


def _pool_dims(k_shape, v_shape, q, page_table_tensor, dev, what):
    """(B, n_groups, S, r_k, r_v, page table or None, page_size, n_pages) of contiguous caches
    [B, G, S, r] or paged pools [n_pages, G, page_size, r] with a [B, max_pages] page table."""
    if page_table_tensor is None:
        B, G, S, r_k = k_shape
        _require(tuple(v_shape[:3]) == (B, G, S), f"v {v_shape} does not match k {k_shape} in [B, {what}, S]")
        return B, G, S, r_k, v_shape[3], None, 0, 0
    n_pages, G, page_size, r_k = k_shape
    _require(tuple(v_shape[:3]) == (n_pages, G, page_size),
             f"v pool {v_shape} does not match k pool {k_shape} in [n_pages, {what}, page_size]")
    B = q.shape[1]
    pt = _page_table(page_table_tensor, B, dev)
    return B, G, pt.shape[1] * page_size, r_k, v_shape[3], pt, page_size, n_pages


def palu_sdpa_decode(q, k_latent, w_rot, cs_tab, v_latent, head_dim_v, cur_pos_tensor, *, rot_step=None,
                     trans_mat=None, u_v=None, scale=None, heads_per_core=None, rot_mode="dst", table_mcast=True,
                     program_config=None, compute_kernel_config=None, memory_config=None,
                     out_dtype=torch.bfloat16, out=None, workspace=None, deterministic=False,
                     page_table_tensor=None, noalloc=False, group_ranks=None, tiled_rows=False) -> torch.Tensor:
    """Fused latent flash-decode (ttnn.transformer.palu_sdpa_decode). Returns [1, B, n_q, head_dim_v], or
    with tiled_rows (bf16, B <= 64; no counterpart in the reference op) a [64, n_q * head_dim_v] buffer in
    the tiled activation layout that the decode step's output projection reads
    (decoder_ops.linear_tiled(..., x_tiled=True)).

    For every p <= cur_pos[b]: K[p] = RoPE_p(k_latent[p] @ u_k) with u_k = w_rot[..., :128], then
    softmax(q K^T * scale) over the attended rows of v_latent (absorbed V). Query head h reads KV head
    h // (n_q // n_kv); KV head j reads latent group j // (n_kv // n_groups).

    compute_kernel_config and memory_config are accepted for call compatibility and unused (the kernel
    always accumulates in fp32; the output is a fresh tensor unless ``out`` is given).
    page_table_tensor [B, max_pages] int32 switches to paged caches: k_latent / v_latent are then page
    pools [n_pages, n_groups, page_size, r] (tensors or LatentCache pools) and position p of row b lives
    on page page_table[b, p // page_size] (ttnn's paged decode convention).
    deterministic=True fixes which wave of a workgroup sums which 32-position block, so repeated calls
    are bit-identical; the default hands blocks out from a counter (faster; calls differ at the bf16
    rounding of the softmax probabilities, well inside the parity tolerance).
    group_ranks=(ranks_k, ranks_v), one rank per latent group (with u_v): each group's own widths, the
    cache columns past them being padding that the kernels never read (the reference pads every group to
    the layer's widest and reads the padding). k_latent / v_latent may also be GroupedLatentCache pairs,
    each group stored at its own ranks (no padding in memory either); their ranks are the group ranks.
    noalloc=True (contiguous caches only, no workspace) calls palu_sdpa_decode_noalloc, which keeps the
    kernels' scratch in the library's static per-GPU array: with ``out`` given, the call allocates no
    device memory at all (for HIP graph capture and serving loops); calls overlapping on one GPU race.
    """
    del compute_kernel_config, memory_config
    _require(isinstance(q, torch.Tensor) and q.dim() == 4 and q.shape[0] == 1 and q.shape[3] == HEAD_DIM,
             f"q must be [1, B, n_q, {HEAD_DIM}], got {tuple(getattr(q, 'shape', ()))}")
    dev = q.device
    _as_dev(q, "q", torch.bfloat16)
    k_store, k_shape, layout = _cache_arg(k_latent, "k_latent", dev, "k")
    v_store, v_shape, v_layout = _cache_arg(v_latent, "v_latent", dev, "v")
    _require(layout == v_layout, "k_latent and v_latent must use the same cache layout")
    B, n_groups, S, r_k, r_v, pt, page_size, n_pages = _pool_dims(k_shape, v_shape, q, page_table_tensor, dev,
                                                                 "n_groups")
    _require(q.shape[1] == B, f"q has batch {q.shape[1]} but the latent caches have {B}")
    n_q = q.shape[2]
    w = w_rot.reshape(-1, *w_rot.shape[-2:]) if w_rot.dim() >= 3 else w_rot
    _require(w.dim() == 3 and (w_rot.dim() == 3 or w_rot.shape[0] == 1),
             f"w_rot must be [1, n_kv, r_k, 256], got {tuple(w_rot.shape)}")
    _as_dev(w, "w_rot", torch.bfloat16, dev)
    n_kv, w_rank, w_width = w.shape
    _require(w_rank == r_k, f"w_rot rank {w_rank} != k_latent width r_k {r_k}")
    cs = cs_tab.reshape(-1, cs_tab.shape[-1])
    _require(cs_tab.dim() in (2, 4), f"cs_tab must be [1, 1, S, 256], got {tuple(cs_tab.shape)}")
    _require(cs.dtype in (torch.float32, torch.bfloat16), f"cs_tab must be fp32 or bf16, got {cs.dtype}")
    _as_dev(cs, "cs_tab", None, dev)
    rot = ROT_MODES.get(rot_mode, -1) if isinstance(rot_mode, str) else -1
    if rot < 0:
        raise RuntimeError(f"rot_mode must be 'legacy', 'pack' or 'dst', got {rot_mode!r}")
    if heads_per_core is not None and int(heads_per_core) > 1 and program_config is not None:
        cores = _grid_cores(program_config)
        hpg = n_kv // n_groups if n_groups and n_kv % n_groups == 0 else 1
        if cores is not None and hpg > 1 and int(heads_per_core) <= n_kv and hpg % int(heads_per_core) == 0:
            items = B * (n_kv // int(heads_per_core))
            _require(items <= cores, f"heads_per_core={heads_per_core} needs {items} cores for {B} rows of "
                                     f"{n_kv // int(heads_per_core)} head groups, only {cores} available")
    if out_dtype not in _DTYPES:
        raise RuntimeError(f"out_dtype must be torch.float32 or torch.bfloat16, got {out_dtype}")
    cp = _cur_pos(cur_pos_tensor, B, dev)
    rs = None if rot_step is None else _as_dev(rot_step.float().contiguous(), "rot_step", torch.float32, dev)
    tm = None if trans_mat is None else _as_dev(trans_mat.contiguous(), "trans_mat", None, dev)
    uv = None if u_v is None else _as_dev(u_v.reshape(-1, *u_v.shape[-2:]).contiguous(), "u_v", torch.bfloat16, dev)
    width = int(head_dim_v)
    od = _DTYPES[out_dtype]
    if tiled_rows:
        _require(out_dtype == torch.bfloat16 and B <= 64, "a tiled-rows output is bf16 for at most 64 rows")
        od |= _native.OUT_TILED_ROWS
        if out is None:
            out = torch.empty(64, n_q * width, dtype=out_dtype, device=dev)
        _as_dev(out, "out", out_dtype, dev)
        _require(tuple(out.shape) == (64, n_q * width) and out.is_contiguous(), f"out must be [64, {n_q * width}]")
    elif out is None:
        out = torch.empty(1, B, n_q, width, dtype=out_dtype, device=dev)
    else:
        _as_dev(out, "out", out_dtype, dev)
        _require(tuple(out.shape) == (1, B, n_q, width), f"out must be [1, {B}, {n_q}, {width}]")
    gr = None
    if layout == _native.LAYOUT_TILED_GROUPED:
        # compact grouped caches carry their groups' ranks; group_ranks, when given, must agree
        cache_ranks = [list(k_latent.ranks), list(v_latent.ranks)]
        _require(group_ranks is None or [[int(r) for r in x] for x in group_ranks] == cache_ranks,
                 f"group_ranks {group_ranks} differ from the GroupedLatentCache ranks {cache_ranks}")
        group_ranks = cache_ranks
    if group_ranks is not None:
        gk, gv = (list(x) for x in group_ranks)
        _require(len(gk) == n_groups and len(gv) == n_groups,
                 f"group_ranks must give {n_groups} K ranks and {n_groups} V ranks")
        _require(pt is None, "group_ranks: per-group ranks are built for contiguous caches")
        gr = (ctypes.c_int32 * (2 * n_groups))(*[int(r) for r in gk + gv])
    lib = _native.load()
    sc = float(HEAD_DIM ** -0.5 if scale is None else scale)
    if noalloc:
        _require(pt is None and workspace is None, "noalloc takes contiguous caches and no workspace")
        _native.check(lib.palu_sdpa_decode_noalloc(
            _native.ptr(q), _native.ptr(k_store), _native.ptr(w), _native.ptr(cs), _native.ptr(v_store), width,
            _native.ptr(cp), _native.ptr(out), _native.ptr(rs), _native.ptr(tm), _native.ptr(uv), gr, sc,
            int(heads_per_core or 0), rot, int(bool(table_mcast)), _k_chunk(program_config), B, n_q, n_kv, n_groups,
            S, r_k, r_v, w_width, cs.shape[0], cs.shape[1], _DTYPES[cs.dtype], od, layout,
            int(bool(deterministic)), _native.stream_handle(dev)))
        return out
    if uv is not None and pt is None:
        ws, ws_bytes = _glrd_workspace(B, n_q, n_kv, n_groups, S, r_v, dev, workspace)
    else:
        ws, ws_bytes = _workspace(B, n_kv, S, max(width, 1), dev, workspace)
    if pt is None:
        _native.check(lib.palu_sdpa_decode(
            _native.ptr(q), _native.ptr(k_store), _native.ptr(w), _native.ptr(cs), _native.ptr(v_store), width,
            _native.ptr(cp), _native.ptr(out), _native.ptr(rs), _native.ptr(tm), _native.ptr(uv), gr, sc,
            int(heads_per_core or 0), rot, int(bool(table_mcast)), _k_chunk(program_config), B, n_q, n_kv, n_groups,
            S, r_k, r_v, w_width, cs.shape[0], cs.shape[1], _DTYPES[cs.dtype], od, layout,
            int(bool(deterministic)), _native.ptr(ws), ws_bytes, _native.stream_handle(dev)))
    else:
        _native.check(lib.palu_sdpa_decode_paged(
            _native.ptr(q), _native.ptr(k_store), _native.ptr(w), _native.ptr(cs), _native.ptr(v_store), width,
            _native.ptr(cp), _native.ptr(pt), _native.ptr(out), _native.ptr(rs), _native.ptr(tm), _native.ptr(uv), sc,
            int(heads_per_core or 0), rot, int(bool(table_mcast)), _k_chunk(program_config), B, n_q, n_kv, n_groups,
            n_pages, page_size, pt.shape[1], r_k, r_v, w_width, cs.shape[0], cs.shape[1], _DTYPES[cs.dtype],
            od, layout, int(bool(deterministic)), _native.ptr(ws), ws_bytes, _native.stream_handle(dev)))
    return out


def flash_decode(q, k, v, cur_pos_tensor, *, scale=None, head_dim_v=None, out_dtype=torch.bfloat16, out=None,
                 workspace=None, deterministic=False, page_table_tensor=None) -> torch.Tensor:
    """Stock flash-decode over full rotated K [B, n_kv, S, 128] and V [B, n_kv, S, head_dim_v]: the
    MI355X counterpart of ttnn.transformer.scaled_dot_product_attention_decode (head_dim_v 128) and
    flash_multi_latent_attention_decode (head_dim_v = V width). Returns [1, B, n_q, head_dim_v].
    With page_table_tensor, k and v are page pools [n_pages, n_kv, page_size, width] (ttnn's
    paged_scaled_dot_product_attention_decode)."""
    _require(isinstance(q, torch.Tensor) and q.dim() == 4 and q.shape[0] == 1 and q.shape[3] == HEAD_DIM,
             f"q must be [1, B, n_q, {HEAD_DIM}]")
    dev = q.device
    _as_dev(q, "q", torch.bfloat16)
    k_store, k_shape, layout = _cache_arg(k, "k", dev, "k")
    v_store, v_shape, v_layout = _cache_arg(v, "v", dev, "v")
    _require(layout == v_layout, "k and v must use the same cache layout")
    B, n_kv, S, hd, v_width, pt, page_size, n_pages = _pool_dims(k_shape, v_shape, q, page_table_tensor, dev, "n_kv")
    _require(hd == HEAD_DIM, f"k must be [B, n_kv, S, {HEAD_DIM}], got {k_shape}")
    _require(q.shape[1] == B, f"q has batch {q.shape[1]} but the caches have {B}")
    width = int(v_width if head_dim_v is None else head_dim_v)
    _require(width == v_width, f"head_dim_v {width} != V width {v_width}")
    n_q = q.shape[2]
    if out_dtype not in _DTYPES:
        raise RuntimeError(f"out_dtype must be torch.float32 or torch.bfloat16, got {out_dtype}")
    cp = _cur_pos(cur_pos_tensor, B, dev)
    if out is None:
        out = torch.empty(1, B, n_q, width, dtype=out_dtype, device=dev)
    ws, ws_bytes = _workspace(B, n_kv, S, width, dev, workspace)
    lib = _native.load()
    sc = float(HEAD_DIM ** -0.5 if scale is None else scale)
    if pt is None:
        _native.check(lib.palu_flash_decode(
            _native.ptr(q), _native.ptr(k_store), _native.ptr(v_store), _native.ptr(cp), _native.ptr(out), sc, B, n_q,
            n_kv, S, width, _DTYPES[out_dtype], layout, int(bool(deterministic)), _native.ptr(ws), ws_bytes,
            _native.stream_handle(dev)))
    else:
        _native.check(lib.palu_flash_decode_paged(
            _native.ptr(q), _native.ptr(k_store), _native.ptr(v_store), _native.ptr(cp), _native.ptr(pt),
            _native.ptr(out), sc, B, n_q, n_kv, n_pages, page_size, pt.shape[1], width, _DTYPES[out_dtype], layout,
            int(bool(deterministic)), _native.ptr(ws), ws_bytes, _native.stream_handle(dev)))
    return out


def scaled_dot_product_attention_decode(q, k, v, cur_pos_tensor, scale=None, **_):
    """Name-compatible alias of the stock decode op (full K and V, head_dim_v = 128)."""
    return flash_decode(q, k, v, cur_pos_tensor, scale=scale)


def flash_multi_latent_attention_decode(q, k, v, head_dim_v, cur_pos_tensor, scale=None, **_):
    """Name-compatible alias of the MLA decode op (full rotated K, V of width head_dim_v)."""
    return flash_decode(q, k, v, cur_pos_tensor, scale=scale, head_dim_v=head_dim_v)


def paged_scaled_dot_product_attention_decode(q, k, v, cur_pos_tensor, page_table_tensor, scale=None, **_):
    """Name-compatible alias of the paged stock decode op (page pools of full K and V)."""
    return flash_decode(q, k, v, cur_pos_tensor, scale=scale, page_table_tensor=page_table_tensor)


def paged_update_cache(cache, new_rows: torch.Tensor, update_idxs_tensor: torch.Tensor, page_table=None) -> None:
    """Latent append (ttnn.experimental.paged_update_cache on a latent cache, attention.py:622-623):
    cache[b, g, update_idxs[b], :] = new_rows[..., b, g, :] for every b with 0 <= idx < S. ``cache`` is a
    [B, G, S, width] bf16 tensor or a LatentCache. With ``page_table`` [B, max_pages] int32 the cache is a
    page pool [n_pages, G, page_size, width] and row b goes to page page_table[b, idx // page_size]."""
    dev = cache.device
    if isinstance(cache, GroupedLatentCache):
        _require(page_table is None, "a GroupedLatentCache is contiguous")
        B, G, S, width = cache.shape
        decoder_ops.append_from(cache, new_rows.reshape(B, G * width), width, width, update_idxs_tensor)
        return
    store, (N, G, S, width), layout = _cache_arg(cache, "cache", dev)
    lib = _native.load()
    if page_table is None:
        B = N
        rows = new_rows.reshape(B, G, width)
        _as_dev(rows, "new_rows", torch.bfloat16, dev)
        cp = _cur_pos(update_idxs_tensor, B, dev)
        _native.check(lib.palu_latent_append(_native.ptr(store), _native.ptr(rows), _native.ptr(cp), B, G, S, width,
                                             layout, _native.stream_handle(dev)))
        return
    B = update_idxs_tensor.numel()
    rows = new_rows.reshape(B, G, width)
    _as_dev(rows, "new_rows", torch.bfloat16, dev)
    cp = _cur_pos(update_idxs_tensor, B, dev)
    pt = _page_table(page_table, B, dev)
    _native.check(lib.palu_latent_append_paged(_native.ptr(store), _native.ptr(rows), _native.ptr(cp), _native.ptr(pt),
                                               B, G, N, S, pt.shape[1], width, layout, _native.stream_handle(dev)))
