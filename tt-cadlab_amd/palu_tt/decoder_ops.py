"""Fused decoder-step ops on MI355X (C-ABI decoder helpers of libpalu_mi355x.so).

They replace the chains of small PyTorch kernels around the decode op: RMSNorm with the residual add,
the SwiGLU gate, RoPE read straight out of the fused QKV projection, and the latent append from the
projection's latent columns. Every op writes into tensors the caller passes or a fresh one; all tensors
are bf16 on the GPU except the fp32 RoPE tables and int32 positions. No CPU fallback: a missing library
raises RuntimeError.
"""
from typing import Optional

import torch

from palu_tt import _native
from palu_tt.cache import LatentCache


def _check(t: torch.Tensor, name: str, dtype=torch.bfloat16) -> None:
    if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == dtype):
        raise RuntimeError(f"{name} must be a {dtype} tensor on the GPU")


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, res: Optional[torch.Tensor] = None,
            h_out: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = h * rsqrt(mean(h^2) + eps) * weight per row with h = x + res (bf16 residual stream; res may be
    None). When h_out is given, h is written there (it may alias x). x, res, h_out, out: [rows, dim]."""
    _check(x, "x")
    _check(weight, "weight")
    rows, dim = x.reshape(-1, x.shape[-1]).shape
    out = torch.empty_like(x) if out is None else out
    for t, n in ((res, "res"), (h_out, "h_out"), (out, "out")):
        if t is not None:
            _check(t, n)
            if t.numel() != x.numel() or not t.is_contiguous():
                raise RuntimeError(f"{n} must be contiguous with the shape of x")
    if not x.is_contiguous():
        raise RuntimeError("x must be contiguous")
    _native.check(_native.load().palu_rmsnorm(
        _native.ptr(x), _native.ptr(res), _native.ptr(h_out), _native.ptr(out), _native.ptr(weight), rows, dim,
        float(eps), _native.stream_handle(x.device)))
    return out


def swiglu(gu: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """silu(g) * u for gu = [g | u] of shape [rows, 2 ffn]; returns [rows, ffn]."""
    _check(gu, "gu")
    if not gu.is_contiguous():
        raise RuntimeError("gu must be contiguous")
    rows, two_f = gu.reshape(-1, gu.shape[-1]).shape
    ffn = two_f // 2
    if out is None:
        out = torch.empty(*gu.shape[:-1], ffn, dtype=torch.bfloat16, device=gu.device)
    _native.check(_native.load().palu_swiglu(_native.ptr(gu), _native.ptr(out), rows, ffn,
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
    src [B, >= ...] (the latent columns of the QKV output). cache: LatentCache (tiled) or a row-major
    [B, G, S, width] bf16 tensor."""
    _check(src, "src")
    if src.dim() != 2 or src.stride(1) != 1:
        raise RuntimeError("src must be a row-strided [rows, width] view")
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
    p = pos.reshape(-1).to(device=src.device, dtype=torch.int32).contiguous()
    _native.check(_native.load().palu_latent_append_strided(
        _native.ptr(store), _native.ptr(src), src.stride(0), int(group_stride), _native.ptr(p), B, G, S, width, layout,
        _native.stream_handle(src.device)))
