"""The decoder-step helpers (palu_tt.decoder_ops over the C-ABI) against plain PyTorch fp32 references
of the same ops: RMSNorm with the residual add, SwiGLU, RoPE of head rows read from a strided QKV
output, and the strided latent append (bit-exact against the contiguous append of the same rows).
Outputs are bf16, so the floating-point bar is one bf16 rounding: |out - ref| <= 1e-2 * (|ref| + 1)."""
import pytest
import torch
import torch.nn.functional as F

from palu_tt import decoder_ops, fused
from palu_tt.cache import LatentCache

pytestmark = pytest.mark.gpu


def _close(out, ref):
    out, ref = out.float().cpu(), ref.float().cpu()
    err = ((out - ref).abs() / (ref.abs() + 1.0)).max().item()
    assert err <= 1e-2, f"max relative error {err:.3e}"


@pytest.mark.parametrize("rows,dim,with_res", [(64, 4096, True), (3, 512, False), (7, 8192, True), (1, 24, True)])
def test_rmsnorm_matches_torch(gpu, rows, dim, with_res):
    g = torch.Generator().manual_seed(rows + dim)
    x = torch.randn(rows, dim, generator=g).to(torch.bfloat16)
    res = torch.randn(rows, dim, generator=g).to(torch.bfloat16) if with_res else None
    w = (1 + 0.1 * torch.randn(dim, generator=g)).to(torch.bfloat16)
    h_ref = (x.float() + res.float()).to(torch.bfloat16) if with_res else x
    hf = h_ref.float()
    y_ref = (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-5) * w.float()).to(torch.bfloat16)
    xd = x.to(gpu)
    y = decoder_ops.rmsnorm(xd, w.to(gpu), 1e-5, res=None if res is None else res.to(gpu), h_out=xd)
    torch.cuda.synchronize()
    assert torch.equal(xd.cpu(), h_ref)                      # residual stream updated in place, bf16-rounded
    _close(y, y_ref)


@pytest.mark.parametrize("rows,ffn", [(64, 14336), (5, 24)])
def test_swiglu_matches_torch(gpu, rows, ffn):
    g = torch.Generator().manual_seed(ffn)
    gu = (3 * torch.randn(rows, 2 * ffn, generator=g)).to(torch.bfloat16)
    ref = (F.silu(gu[:, :ffn].float()) * gu[:, ffn:].float()).to(torch.bfloat16)
    out = decoder_ops.swiglu(gu.to(gpu))
    torch.cuda.synchronize()
    _close(out, ref)


def test_rope_rows_matches_apply_rope_meta(gpu):
    g = torch.Generator().manual_seed(5)
    B, nh, nkv, S = 6, 32, 8, 2304
    cos, sin = fused.cos_sin_tables(128, S, 500000.0, {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                                                       "high_freq_factor": 4.0, "original_max_position_embeddings": 8192})
    xqkv = torch.randn(B, (nh + 2 * nkv) * 128, generator=g).to(torch.bfloat16)
    pos = torch.tensor([0, 1, 31, 2047, 2303, 977], dtype=torch.int32)
    q_ref = fused.apply_rope_meta(xqkv[:, :nh * 128].float().view(B, nh, 128), cos[pos.long()][:, None], sin[pos.long()][:, None])
    k_ref = fused.apply_rope_meta(xqkv[:, nh * 128:(nh + nkv) * 128].float().view(B, nkv, 128), cos[pos.long()][:, None],
                                  sin[pos.long()][:, None])
    xd, cd, sd, pd = xqkv.to(gpu), cos.to(gpu), sin.to(gpu), pos.to(gpu)
    q = decoder_ops.rope_rows(xd, nh, pd, cd, sd)
    k = decoder_ops.rope_rows(xd[:, nh * 128:], nkv, pd, cd, sd)      # strided view of the K columns
    torch.cuda.synchronize()
    _close(q, q_ref.to(torch.bfloat16))
    _close(k, k_ref.to(torch.bfloat16))


@pytest.mark.parametrize("layout,role,gs,width", [("tiled", "k", 1, 64), ("tiled", "v", 1, 96), ("rows", "k", 1, 32),
                                                   ("tiled", "k", 4, 384), ("tiled", "v", 2, 256), ("rows", "v", 4, 512)])
def test_strided_append_equals_contiguous_append(gpu, layout, role, gs, width):
    g = torch.Generator().manual_seed(width + gs)
    B, nkv, S = 5, 8, 96
    G = nkv // gs
    cols = torch.randn(B, nkv * 128 + 64, generator=g).to(torch.bfloat16).to(gpu)   # extra columns past the slots
    pos = torch.tensor([0, 95, 33, 64, 7], dtype=torch.int32).to(gpu)
    rows = torch.stack([cols[:, gi * gs * 128: gi * gs * 128 + width] for gi in range(G)], dim=1).contiguous()
    make = (lambda: LatentCache.zeros(B, G, S, width, gpu, role)) if layout == "tiled" else \
        (lambda: torch.zeros(B, G, S, width, dtype=torch.bfloat16, device=gpu))
    a, b = make(), make()
    fused.paged_update_cache(a, rows, pos)
    decoder_ops.append_from(b, cols, gs * 128, width, pos)
    torch.cuda.synchronize()
    ta = a.data if layout == "tiled" else a
    tb = b.data if layout == "tiled" else b
    assert torch.equal(ta, tb)
