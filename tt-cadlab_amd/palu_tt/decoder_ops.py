"""Fused decoder-step ops on MI355X (C-ABI decoder helpers of libpalu_mi355x.so).

They replace the chains of small PyTorch kernels around the decode op: RMSNorm with the residual add,
the SwiGLU gate, RoPE read straight out of the fused QKV projection, and the latent append from the
projection's latent columns. Every op writes into tensors the caller passes or a fresh one; all tensors
are bf16 on the GPU except the fp32 RoPE tables and int32 positions. No CPU fallback: a missing library
raises RuntimeError.
"""
import ctypes
from typing import Optional

import torch

from palu_tt import _native
from palu_tt.cache import GroupedLatentCache, LatentCache


def _check(t: torch.Tensor, name: str, dtype=torch.bfloat16) -> None:
    if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == dtype):
        raise RuntimeError(f"{name} must be a {dtype} tensor on the GPU")


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, res: Optional[torch.Tensor] = None,
            h_out: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
            tiled_out: bool = False, res_part: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = h * rsqrt(mean(h^2) + eps) * weight per row with h = x + res (bf16 residual stream; res may be
    None), or h = x + the sum of res_part (fp32 [ks, rows, dim], a projection's split partials, from
    linear_tiled(..., mode="partials")). When h_out is given, h is written there (it may alias x). x, res,
    h_out: [rows, dim]; out: [rows, dim], or with tiled_out a [64, dim] buffer in the tiled activation
    layout (tile_rows) that linear_tiled(..., x_tiled=True) reads (rows <= 64)."""
    _check(x, "x")
    _check(weight, "weight")
    rows, dim = x.reshape(-1, x.shape[-1]).shape
    ks = 0
    if res_part is not None:
        _check(res_part, "res_part", torch.float32)
        if res_part.dim() != 3 or res_part.shape[1:] != (rows, dim) or not res_part.is_contiguous():
            raise RuntimeError(f"res_part must be a contiguous [ks, {rows}, {dim}] fp32 tensor")
        ks = res_part.shape[0]
    if out is None:
        out = (torch.empty(64, dim, dtype=torch.bfloat16, device=x.device) if tiled_out else torch.empty_like(x))
    for t, n in ((res, "res"), (h_out, "h_out")):
        if t is not None:
            _check(t, n)
            if t.numel() != x.numel() or not t.is_contiguous():
                raise RuntimeError(f"{n} must be contiguous with the shape of x")
    _check(out, "out")
    if not out.is_contiguous() or out.numel() != (64 * dim if tiled_out else x.numel()):
        raise RuntimeError("out must be contiguous with the shape of x ([64, dim] when tiled)")
    if not x.is_contiguous():
        raise RuntimeError("x must be contiguous")
    _native.check(_native.load().palu_rmsnorm(
        _native.ptr(x), _native.ptr(res), _native.ptr(res_part), ks, _native.ptr(h_out), _native.ptr(out),
        _native.ptr(weight), rows, dim, float(eps), int(tiled_out), _native.stream_handle(x.device)))
    return out


def argmax_rows(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """torch.argmax(x, dim=-1) of a bf16 [rows, n] tensor (row-strided, stride a multiple of 8) as int64
    [rows]: the first index among equal maxima, NaN above every number."""
    _check(x, "x")
    if x.dim() != 2 or x.stride(1) != 1:
        raise RuntimeError("x must be a row-strided [rows, n] bf16 view")
    rows, n = x.shape
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=x.device)
    if out.dtype != torch.int64 or out.shape != (rows,) or not out.is_contiguous() or out.device != x.device:
        raise RuntimeError(f"out must be a contiguous int64 [{rows}] tensor on {x.device}")
    _native.check(_native.load().palu_argmax_rows(_native.ptr(x), x.stride(0), rows, n, _native.ptr(out),
                                                  _native.stream_handle(x.device)))
    return out


def swiglu(gu: torch.Tensor, out: Optional[torch.Tensor] = None, tiled_out: bool = False) -> torch.Tensor:
    """silu(g) * u for gu = [g | u] of shape [rows, 2 ffn]; returns [rows, ffn], or with tiled_out a
    [64, ffn] buffer in the tiled activation layout (rows <= 64)."""
    _check(gu, "gu")
    if not gu.is_contiguous():
        raise RuntimeError("gu must be contiguous")
    rows, two_f = gu.reshape(-1, gu.shape[-1]).shape
    ffn = two_f // 2
    if out is None:
        out = (torch.empty(64, ffn, dtype=torch.bfloat16, device=gu.device) if tiled_out
               else torch.empty(*gu.shape[:-1], ffn, dtype=torch.bfloat16, device=gu.device))
    _native.check(_native.load().palu_swiglu(_native.ptr(gu), _native.ptr(out), rows, ffn, int(tiled_out),
                                             _native.stream_handle(gu.device)))
    return out


def rope_rows(src: torch.Tensor, heads: int, pos: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Meta-interleaved RoPE of the first `heads` 128-wide heads of every row of src ([rows, >= heads *
    128], a row-strided view such as a column slice of the QKV output) at pos[row]; returns
    [rows, heads, 128]. cos / sin: fp32 [table_rows, 128] (fused.cos_sin_tables)."""
    _check(src, "src")
    _check(cos, "cos", torch.float32)
    _check(sin, "sin", torch.float32)
    if src.dim() != 2 or src.stride(1) != 1:
        raise RuntimeError("src must be a row-strided [rows, width] view")
    rows = src.shape[0]
    p = pos.reshape(-1).to(device=src.device, dtype=torch.int32).contiguous()
    if p.numel() != rows:
        raise RuntimeError(f"pos has {p.numel()} entries for {rows} rows")
    if out is None:
        out = torch.empty(rows, heads, 128, dtype=torch.bfloat16, device=src.device)
    _native.check(_native.load().palu_rope_rows(
        _native.ptr(src), src.stride(0), _native.ptr(out), _native.ptr(p), _native.ptr(cos), _native.ptr(sin),
        cos.shape[0], rows, heads, _native.stream_handle(src.device)))
    return out


def append_from(cache, src: torch.Tensor, group_stride: int, width: int, pos: torch.Tensor) -> None:
    """cache[b, g, pos[b], :] = src[b, g * group_stride : g * group_stride + width] for a row-strided
    src [B, >= ...] (the latent columns of the QKV output). cache: LatentCache (tiled), a row-major
    [B, G, S, width] bf16 tensor, or a GroupedLatentCache (each group takes its first ranks[g] columns)."""
    _check(src, "src")
    if src.dim() != 2 or src.stride(1) != 1:
        raise RuntimeError("src must be a row-strided [rows, width] view")
    p = pos.reshape(-1).to(device=src.device, dtype=torch.int32).contiguous()
    if isinstance(cache, GroupedLatentCache):
        # each group's first ranks[g] columns of its width-wide source slice
        B, G, S, w = cache.shape
        if w > width:
            raise RuntimeError(f"cache ranks up to {w} exceed the append width {width}")
        widths = (ctypes.c_int32 * G)(*cache.ranks)
        order = _native.LAYOUT_TILED if cache.role == "k" else _native.LAYOUT_TILED_V
        _native.check(_native.load().palu_latent_append_grouped(
            _native.ptr(cache.data), _native.ptr(src), src.stride(0), int(group_stride), _native.ptr(p), B, G, S, widths,
            order, _native.stream_handle(src.device)))
        return
    if isinstance(cache, LatentCache):
        store = cache.data
        B, G, S, w = cache.shape
        layout = _native.LAYOUT_TILED if cache.role == "k" else _native.LAYOUT_TILED_V
    else:
        store = cache
        B, G, S, w = cache.shape
        layout = _native.LAYOUT_ROWS
    if w != width:
        raise RuntimeError(f"cache width {w} != append width {width}")
    _native.check(_native.load().palu_latent_append_strided(
        _native.ptr(store), _native.ptr(src), src.stride(0), int(group_stride), _native.ptr(p), B, G, S, width, layout,
        _native.stream_handle(src.device)))


def tile_weight(w: torch.Tensor, rtw: int) -> torch.Tensor:
    """The [n, k] nn.Linear weight in the decode projection's tiled order for workgroups of rtw row tiles
    (a new contiguous tensor of the same bytes). Tile (rt, kt) of 16 output columns x 32 inputs is 1 KB,
    lane 16 g + i holding w[16 rt + i][32 kt + 8 g .. +7]. Row tiles form groups of rtw (the last group
    may be shorter); inside a group the tiles are stored k tile by k tile, [kt][rt in group], so the
    workgroup that owns a group reads it as one sequential stream. n a multiple of 16, k of 32."""
    n, k = w.shape
    if n % 16 or k % 32:
        raise RuntimeError(f"tile_weight: shape [{n}, {k}] needs n % 16 == 0 and k % 32 == 0")
    if not 1 <= rtw <= 8:
        raise RuntimeError(f"tile_weight: rtw = {rtw} must be in 1..8")
    n16, kt = n // 16, k // 32
    t = w.reshape(n16, 16, kt, 4, 8).permute(0, 2, 3, 1, 4)               # [rt, kt, g, i, e]
    full = (n16 // rtw) * rtw
    parts = [t[:full].reshape(n16 // rtw, rtw, kt, 4, 16, 8).transpose(1, 2).reshape(-1)]
    if full < n16:
        parts.append(t[full:].transpose(0, 1).reshape(-1))
    return torch.cat(parts).reshape(n, k)


def untile_weight(wt: torch.Tensor, rtw: int) -> torch.Tensor:
    """Inverse of tile_weight: the [n, k] nn.Linear layout."""
    n, k = wt.shape
    n16, kt = n // 16, k // 32
    full = (n16 // rtw) * rtw
    flat = wt.reshape(-1)
    t = flat[:full * kt * 512].reshape(n16 // rtw, kt, rtw, 4, 16, 8).transpose(1, 2).reshape(full, kt, 4, 16, 8)
    if full < n16:
        rest = flat[full * kt * 512:].reshape(kt, n16 - full, 4, 16, 8).transpose(0, 1)
        t = torch.cat([t, rest])
    return t.permute(0, 3, 1, 2, 4).reshape(n, k).contiguous()


def tile_rows(x: torch.Tensor) -> torch.Tensor:
    """Activations [rows <= 64, k] in the 64-row tiled layout that linear_tiled reads with x_tiled=True
    (rows padded with zeros to 64, then tile_weight's order with the four 16-row tiles as one group)."""
    rows, k = x.shape
    if rows > 64:
        raise RuntimeError(f"tile_rows: {rows} rows (at most 64)")
    pad = torch.zeros(64, k, dtype=x.dtype, device=x.device)
    pad[:rows] = x
    return tile_weight(pad, 4)


def untile_rows(xt: torch.Tensor, rows: int) -> torch.Tensor:
    """Inverse of tile_rows: the first `rows` rows of a [64, k] tiled activation buffer, row-major."""
    return untile_weight(xt, 4)[:rows]


def linear_plan(rows: int, n: int, k: int, max_ks: int = 16):
    """(row tiles per workgroup, k slices) suggested for this shape, with at most max_ks slices (1 for the
    fused epilogues: linear_swiglu_rmsnorm, linear_residual, linear_qkv): tile the weight with that rtw."""
    rtw, ks = ctypes.c_int(0), ctypes.c_int(0)
    _native.check(_native.load().palu_linear_plan_ks(rows, n, k, max_ks, ctypes.byref(rtw), ctypes.byref(ks)))
    return rtw.value, ks.value


_LINEAR_MODES = {"bf16": 0, "partials": 1, "swiglu": 2}


def linear_tiled(x: torch.Tensor, w_tiled: torch.Tensor, rtw: int, ks: int, out: Optional[torch.Tensor] = None,
                 workspace: Optional[torch.Tensor] = None, x_tiled: bool = False, rows: Optional[int] = None,
                 mode: str = "bf16") -> torch.Tensor:
    """x @ w.T for the decode step's rows (at most 64) with w given by tile_weight(w, rtw) ([n, k]), split
    into ks k slices. x: a row-strided [rows, k] view, or with x_tiled a [64, k] buffer in the tiled
    activation layout (tile_rows; rmsnorm / swiglu with tiled_out) and `rows` the live row count.
    mode "bf16": returns [rows, n] bf16 (or writes `out`, a row-strided [rows, n] view); split partials
    go to `workspace` (a uint8 GPU tensor of at least palu_linear_workspace_bytes, else a fresh one from
    torch's caching allocator) and a second launch adds them. mode "partials": returns the fp32 split
    partials [ks, rows, n] for a consumer that sums them (rmsnorm's res_part, qkv_post). mode "swiglu": w
    is interleave_gate_up's gate / up weight (ks = 1) and the result is silu(gate) * up as [64, n / 2]
    tiled activations. linear_plan(rows, n, k) suggests (rtw, ks)."""
    _check(x, "x")
    _check(w_tiled, "w_tiled")
    if x.dim() != 2 or x.stride(1) != 1 or w_tiled.dim() != 2 or not w_tiled.is_contiguous():
        raise RuntimeError("x must be a row-strided [rows, k] view and w_tiled a contiguous [n, k] tensor")
    if mode not in _LINEAR_MODES:
        raise RuntimeError(f"mode must be one of {sorted(_LINEAR_MODES)}")
    k = x.shape[1]
    if x_tiled:
        if x.shape[0] != 64 or not x.is_contiguous() or rows is None:
            raise RuntimeError("a tiled x is a contiguous [64, k] buffer and needs the live row count `rows`")
    else:
        rows = x.shape[0]
    n = w_tiled.shape[0]
    if w_tiled.shape[1] != k:
        raise RuntimeError(f"x has k = {k}, w_tiled has {w_tiled.shape[1]}")
    if mode == "partials":
        if out is None:
            out = torch.empty(ks, rows, n, dtype=torch.float32, device=x.device)
        _check(out, "out", torch.float32)
        if out.shape != (ks, rows, n) or not out.is_contiguous():
            raise RuntimeError(f"out must be a contiguous [{ks}, {rows}, {n}] fp32 tensor")
    elif mode == "swiglu":
        if out is None:
            out = torch.empty(64, n // 2, dtype=torch.bfloat16, device=x.device)
        _check(out, "out")
        if out.shape != (64, n // 2) or not out.is_contiguous():
            raise RuntimeError(f"out must be a contiguous [64, {n // 2}] bf16 tensor")
    else:
        if out is None:
            out = torch.empty(rows, n, dtype=torch.bfloat16, device=x.device)
        _check(out, "out")
        if out.dim() != 2 or out.shape != (rows, n) or out.stride(1) != 1:
            raise RuntimeError(f"out must be a row-strided [{rows}, {n}] view")
    lib = _native.load()
    need = lib.palu_linear_workspace_bytes(rows, n, k, ks) if mode == "bf16" else 0
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    _native.check(lib.palu_linear_tiled(
        _native.ptr(x), x.stride(0), int(x_tiled), rows, _native.ptr(w_tiled), n, k, _native.ptr(out),
        out.stride(0) if mode == "bf16" else n, _LINEAR_MODES[mode], rtw, ks,
        _native.ptr(workspace) if need else None, need, _native.stream_handle(x.device)))
    return out


def _operands(x: torch.Tensor, w_tiled: torch.Tensor, x_tiled: bool, rows: Optional[int]):
    """(rows, n, k) of a decode projection's operands, checked as linear_tiled checks them."""
    _check(x, "x")
    _check(w_tiled, "w_tiled")
    if x.dim() != 2 or x.stride(1) != 1 or w_tiled.dim() != 2 or not w_tiled.is_contiguous():
        raise RuntimeError("x must be a row-strided [rows, k] view and w_tiled a contiguous [n, k] tensor")
    if x_tiled:
        if x.shape[0] != 64 or not x.is_contiguous() or rows is None:
            raise RuntimeError("a tiled x is a contiguous [64, k] buffer and needs the live row count `rows`")
    else:
        rows = x.shape[0]
    n, k = w_tiled.shape
    if x.shape[1] != k:
        raise RuntimeError(f"x has k = {x.shape[1]}, w_tiled has {k}")
    return rows, n, k


def linear_swiglu_rmsnorm(x: torch.Tensor, w_tiled: torch.Tensor, rtw: int, eps: float,
                          out: Optional[torch.Tensor] = None, x_tiled: bool = False,
                          rows: Optional[int] = None) -> torch.Tensor:
    """silu(g) * u with g, u the gate / up products of the RMS-normalised rows of x, in one launch: w_tiled
    is tile_weight(interleave_gate_up(w1 * norm_w, w3 * norm_w), rtw) (the norm's weight folded into the
    columns), each row's products scaled by rsqrt(mean(x^2) + eps). Returns (or writes `out`) the
    [64, n / 2] tiled activations of linear_tiled's "swiglu" mode."""
    rows, n, k = _operands(x, w_tiled, x_tiled, rows)
    if out is None:
        out = torch.empty(64, n // 2, dtype=torch.bfloat16, device=x.device)
    _check(out, "out")
    if out.shape != (64, n // 2) or not out.is_contiguous():
        raise RuntimeError(f"out must be a contiguous [64, {n // 2}] bf16 tensor")
    _native.check(_native.load().palu_linear_swiglu_rmsnorm(
        _native.ptr(x), x.stride(0), int(x_tiled), rows, _native.ptr(w_tiled), n, k, rtw, float(eps), _native.ptr(out),
        _native.stream_handle(x.device)))
    return out


def linear_residual(x: torch.Tensor, w_tiled: torch.Tensor, rtw: int, h: torch.Tensor,
                    h_tiled: Optional[torch.Tensor] = None, x_tiled: bool = False,
                    rows: Optional[int] = None) -> torch.Tensor:
    """h += x @ w.T in one launch (h a row-strided bf16 [rows, n] view, updated in place, each value
    rounded once), and the new h written to h_tiled ([64, n] tiled activations) when given. Returns h."""
    rows, n, k = _operands(x, w_tiled, x_tiled, rows)
    _check(h, "h")
    if h.dim() != 2 or h.shape != (rows, n) or h.stride(1) != 1:
        raise RuntimeError(f"h must be a row-strided [{rows}, {n}] view")
    if h_tiled is not None:
        _check(h_tiled, "h_tiled")
        if h_tiled.shape != (64, n) or not h_tiled.is_contiguous():
            raise RuntimeError(f"h_tiled must be a contiguous [64, {n}] bf16 tensor")
    _native.check(_native.load().palu_linear_residual(
        _native.ptr(x), x.stride(0), int(x_tiled), rows, _native.ptr(w_tiled), n, k, rtw, _native.ptr(h), h.stride(0),
        _native.ptr(h_tiled) if h_tiled is not None else None, _native.stream_handle(x.device)))
    return h


def _cache_args(cache):
    """(storage, layout, [B, G, S, width]) of a latent cache: LatentCache (tiled) or a row-major tensor."""
    if isinstance(cache, LatentCache):
        layout = _native.LAYOUT_TILED if cache.role == "k" else _native.LAYOUT_TILED_V
        return cache.data, layout, cache.shape
    return cache, _native.LAYOUT_ROWS, cache.shape


def linear_qkv(x: torch.Tensor, w_tiled: torch.Tensor, rtw: int, pos: torch.Tensor, cos: torch.Tensor,
               sin: torch.Tensor, n_heads: int, keys, k_col_offset: int, k_group_stride: int, k_width: int, values,
               v_col_offset: int, v_group_stride: int, v_width: int, k_rope: bool = False,
               q_out: Optional[torch.Tensor] = None, x_tiled: bool = False,
               rows: Optional[int] = None) -> torch.Tensor:
    """The decode step's QKV projection and its epilogue in one launch: the columns of x @ w.T go where
    qkv_post sends the summed partials (q [B, n_heads, 128] rotated at pos, returned; K / V latent slices
    appended to keys / values at pos), with the same rounding."""
    rows, n, k = _operands(x, w_tiled, x_tiled, rows)
    _check(cos, "cos", torch.float32)
    _check(sin, "sin", torch.float32)
    p = pos.reshape(-1).to(device=x.device, dtype=torch.int32).contiguous()
    if p.numel() != rows:
        raise RuntimeError(f"pos has {p.numel()} entries for {rows} rows")
    if q_out is None:
        q_out = torch.empty(rows, n_heads, 128, dtype=torch.bfloat16, device=x.device)
    kd, kl, (kb, G, S, kw) = _cache_args(keys)
    vd, vl, (vb, vG, vS, vw) = _cache_args(values)
    if (kb, G, S, kw) != (rows, G, S, k_width) or (vb, vG, vS, vw) != (rows, G, S, v_width):
        raise RuntimeError("cache shapes must be [B, G, S, k_width] and [B, G, S, v_width]")
    _native.check(_native.load().palu_linear_qkv(
        _native.ptr(x), x.stride(0), int(x_tiled), rows, _native.ptr(w_tiled), n, k, rtw, _native.ptr(p),
        _native.ptr(cos), _native.ptr(sin), cos.shape[0], n_heads, _native.ptr(q_out), _native.ptr(kd), kl,
        k_col_offset, k_group_stride, k_width, int(k_rope), _native.ptr(vd), vl, v_col_offset, v_group_stride, v_width,
        G, S, _native.stream_handle(x.device)))
    return q_out


def interleave_gate_up(w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """[2 ffn, k] with gate and up rows interleaved eight at a time (rows 16 j .. 16 j + 7: gate rows
    8 j .. 8 j + 7, then the up rows of the same outputs), the weight linear_tiled's "swiglu" mode takes."""
    f, k = w_gate.shape
    if w_up.shape != (f, k) or f % 8:
        raise RuntimeError("gate and up weights must share a shape [ffn, k] with ffn a multiple of 8")
    return torch.stack([w_gate.reshape(f // 8, 8, k), w_up.reshape(f // 8, 8, k)], 1).reshape(2 * f, k)


def deinterleave_gate_up(w: torch.Tensor) -> torch.Tensor:
    """Inverse of interleave_gate_up, as one [2 ffn, k] tensor: the gate rows, then the up rows."""
    f2, k = w.shape
    t = w.reshape(f2 // 16, 2, 8, k)
    return torch.cat([t[:, 0].reshape(f2 // 2, k), t[:, 1].reshape(f2 // 2, k)], 0)


def qkv_post(part: torch.Tensor, pos: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, n_heads: int,
             keys, k_col_offset: int, k_group_stride: int, k_width: int, values, v_col_offset: int,
             v_group_stride: int, v_width: int, k_rope: bool = False,
             q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The QKV epilogue of a decode step in one launch, from the projection's fp32 split partials part
    [ks, B, ncols]: returns q [B, n_heads, 128], the first n_heads heads rotated at pos (as rope_rows), and
    appends every latent group's K and V slices (columns k_col_offset + g * k_group_stride, k_width wide,
    rotated too when k_rope; v_col_offset + g * v_group_stride, v_width wide) to keys / values at pos (as
    append_from). keys / values: LatentCache (tiled) or row-major [B, G, S, width] bf16 tensors."""
    _check(part, "part", torch.float32)
    _check(cos, "cos", torch.float32)
    _check(sin, "sin", torch.float32)
    if part.dim() != 3 or not part.is_contiguous():
        raise RuntimeError("part must be a contiguous [ks, B, ncols] fp32 tensor")
    ks, B, ncols = part.shape
    p = pos.reshape(-1).to(device=part.device, dtype=torch.int32).contiguous()
    if p.numel() != B:
        raise RuntimeError(f"pos has {p.numel()} entries for {B} rows")
    if q_out is None:
        q_out = torch.empty(B, n_heads, 128, dtype=torch.bfloat16, device=part.device)

    kd, kl, (kb, G, S, kw) = _cache_args(keys)
    vd, vl, (vb, vG, vS, vw) = _cache_args(values)
    if (kb, G, S, kw) != (B, G, S, k_width) or (vb, vG, vS, vw) != (B, G, S, v_width):
        raise RuntimeError("cache shapes must be [B, G, S, k_width] and [B, G, S, v_width]")
    _native.check(_native.load().palu_qkv_post(
        _native.ptr(part), ks, B, ncols, _native.ptr(p), _native.ptr(cos), _native.ptr(sin), cos.shape[0], n_heads,
        _native.ptr(q_out), _native.ptr(kd), kl, k_col_offset, k_group_stride, k_width, int(k_rope), _native.ptr(vd),
        vl, v_col_offset, v_group_stride, v_width, G, S, _native.stream_handle(part.device)))
    return q_out


def linear_argmax(x: torch.Tensor, w_tiled: torch.Tensor, rtw: int, workspace: Optional[torch.Tensor] = None,
                  x_tiled: bool = False, rows: Optional[int] = None,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """argmax_rows(linear_tiled(x, w_tiled, rtw, 1)) as int64 [rows] without writing the logits: the
    projection's epilogue keeps each row's largest (value, first column) per group of row tiles and a
    second launch picks among the groups. x as for linear_tiled; workspace: a uint8 GPU tensor of at
    least palu_linear_argmax_workspace_bytes(rows, n) bytes (else a fresh one)."""
    _check(x, "x")
    _check(w_tiled, "w_tiled")
    k = x.shape[1]
    if x_tiled:
        if x.shape[0] != 64 or not x.is_contiguous() or rows is None:
            raise RuntimeError("a tiled x is a contiguous [64, k] buffer and needs the live row count `rows`")
    else:
        rows = x.shape[0]
        if x.dim() != 2 or x.stride(1) != 1:
            raise RuntimeError("x must be a row-strided [rows, k] view")
    n = w_tiled.shape[0]
    if w_tiled.shape[1] != k:
        raise RuntimeError(f"x has k = {k}, w_tiled has {w_tiled.shape[1]}")
    lib = _native.load()
    need = lib.palu_linear_argmax_workspace_bytes(rows, n)
    if workspace is None:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=x.device)
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=x.device)
    if out.dtype != torch.int64 or out.shape != (rows,) or not out.is_contiguous() or out.device != x.device:
        raise RuntimeError(f"out must be a contiguous int64 [{rows}] tensor on {x.device}")
    _native.check(lib.palu_linear_argmax(_native.ptr(x), 64 if x_tiled else x.stride(0), int(x_tiled), rows,
                                         _native.ptr(w_tiled), n, k, rtw, _native.ptr(out), _native.ptr(workspace),
                                         workspace.numel(), _native.stream_handle(x.device)))
    return out


class DecodeLinear:
    """One projection of the decode step, y = x @ w.T, for w [n, k] in the nn.Linear layout (for a gate /
    up pair, gate_up=(w_gate, w_up) instead: y = silu(x @ w_gate.T) * (x @ w_up.T)). For up to 64 rows
    (and n % 16 == 0, k % 32 == 0) the weight is held only in the tiled order of linear_tiled, with the
    work split linear_plan suggests (or rtw / ks; single_slice: one k slice, for the fused residual and
    QKV epilogues) and a workspace for its split partials; otherwise it stays as it is and the call is
    torch's F.linear. plain() returns the weight in the nn.Linear layout ([gate; up] for a pair; a fresh
    copy when tiled), for the prefill's many-row products. in_scale (a gate / up pair only): the weight of
    the RMSNorm in front of the pair, folded into the tiled weight's columns (w * in_scale) so that
    norm_eps calls take the normalisation into the same launch (linear_swiglu_rmsnorm); in_scale_folded
    says whether it was (only a tiled pair folds it), and then plain() holds the folded weight too."""

    def __init__(self, w: Optional[torch.Tensor], rows: int, gate_up=None, rtw: int = 0, ks: int = 0,
                 single_slice: bool = False, in_scale: Optional[torch.Tensor] = None):
        self.gate_up = gate_up is not None
        if self.gate_up:
            w = torch.cat(list(gate_up), 0)
        elif in_scale is not None:
            raise RuntimeError("in_scale is folded into a gate / up pair only")
        n, k = w.shape
        self.n, self.k = n, k
        self.tiled = (rows <= 64 and n % (64 if self.gate_up else 16) == 0 and k % 32 == 0 and w.is_cuda
                      and w.dtype == torch.bfloat16)
        self.in_scale_folded = False
        self.argmax_ws = None
        if self.tiled:
            self.rtw, self.ks = (rtw, ks) if rtw else linear_plan(rows, n, k, 1 if single_slice else 16)
            if self.gate_up:
                self.ks = 1
                g, u = gate_up
                if in_scale is not None:
                    sc = in_scale.float().reshape(1, k)
                    g, u = (g.float() * sc).to(g.dtype), (u.float() * sc).to(u.dtype)
                    self.in_scale_folded = True
                w = interleave_gate_up(g, u)
            self.weight = tile_weight(w, self.rtw)
            need = _native.load().palu_linear_workspace_bytes(rows, n, k, self.ks)
            self.workspace = torch.empty(need, dtype=torch.uint8, device=w.device) if need else None
        else:
            self.ks = 1
            self.weight = w.contiguous()

    def __call__(self, x: torch.Tensor, out: Optional[torch.Tensor] = None, x_tiled: bool = False,
                 rows: Optional[int] = None, mode: Optional[str] = None) -> torch.Tensor:
        """x: [rows, k] (row-strided), or with x_tiled the [64, k] tiled activation buffer and `rows`.
        mode (linear_tiled's): "bf16" (the default of a plain projection), "partials" (fp32 [ks, rows, n]),
        "swiglu" (the default and only mode of a gate / up pair: [64, n / 2] tiled activations when tiled,
        else [rows, n / 2] bf16)."""
        mode = mode or ("swiglu" if self.gate_up else "bf16")
        if (mode == "swiglu") != self.gate_up:
            raise RuntimeError("the swiglu mode is the gate / up pair's only mode")
        if self.tiled:
            return linear_tiled(x, self.weight, self.rtw, self.ks, out=out, workspace=self.workspace,
                                x_tiled=x_tiled, rows=rows, mode=mode)
        if x_tiled:
            raise RuntimeError("tiled activations need a tiled projection (at most 64 rows)")
        y = torch.nn.functional.linear(x, self.weight)
        if mode == "swiglu":
            return swiglu(y)
        if mode == "partials":
            return y.float()[None]
        if out is not None:
            out.copy_(y)
            return out
        return y

    def argmax(self, x: torch.Tensor, x_tiled: bool = False, rows: Optional[int] = None) -> torch.Tensor:
        """argmax_rows(self(x)) as int64 [rows]: linear_argmax for a tiled projection (the logits are not
        written), else torch's projection and argmax_rows."""
        if self.tiled and not self.gate_up:
            if self.argmax_ws is None:
                need = _native.load().palu_linear_argmax_workspace_bytes(64, self.n)
                self.argmax_ws = torch.empty(need, dtype=torch.uint8, device=self.weight.device)
            return linear_argmax(x, self.weight, self.rtw, self.argmax_ws, x_tiled=x_tiled, rows=rows)
        return argmax_rows(self(x, x_tiled=x_tiled, rows=rows))

    def swiglu_rmsnorm(self, x: torch.Tensor, eps: float, out: Optional[torch.Tensor] = None,
                       x_tiled: bool = False, rows: Optional[int] = None) -> torch.Tensor:
        """A folded gate / up pair over the RMS-normalised rows of x (linear_swiglu_rmsnorm): [64, n / 2]
        tiled activations."""
        if not (self.gate_up and self.in_scale_folded):
            raise RuntimeError("swiglu_rmsnorm needs a tiled gate / up pair with the norm weight folded in")
        return linear_swiglu_rmsnorm(x, self.weight, self.rtw, eps, out=out, x_tiled=x_tiled, rows=rows)

    def residual(self, x: torch.Tensor, h: torch.Tensor, h_tiled: Optional[torch.Tensor] = None,
                 x_tiled: bool = False, rows: Optional[int] = None) -> torch.Tensor:
        """h += x @ w.T (linear_residual; a single-slice tiled projection), h_tiled the new h tiled."""
        if not self.tiled or self.ks != 1 or self.gate_up:
            raise RuntimeError("residual needs a tiled single-slice projection")
        return linear_residual(x, self.weight, self.rtw, h, h_tiled, x_tiled=x_tiled, rows=rows)

    def qkv(self, x: torch.Tensor, pos, cos, sin, n_heads, keys, k_col_offset, k_group_stride, k_width, values,
            v_col_offset, v_group_stride, v_width, k_rope=False, x_tiled: bool = False,
            rows: Optional[int] = None) -> torch.Tensor:
        """The QKV projection with its epilogue (linear_qkv; a single-slice tiled projection): returns q."""
        if not self.tiled or self.ks != 1 or self.gate_up:
            raise RuntimeError("qkv needs a tiled single-slice projection")
        return linear_qkv(x, self.weight, self.rtw, pos, cos, sin, n_heads, keys, k_col_offset, k_group_stride,
                          k_width, values, v_col_offset, v_group_stride, v_width, k_rope=k_rope, x_tiled=x_tiled,
                          rows=rows)

    def plain(self) -> torch.Tensor:
        if not self.tiled:
            return self.weight
        w = untile_weight(self.weight, self.rtw)
        return deinterleave_gate_up(w) if self.gate_up else w
