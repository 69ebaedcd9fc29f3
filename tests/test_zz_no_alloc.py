"""palu_sdpa_decode_noalloc through the C-ABI: the allocation-free variant of palu_sdpa_decode, whose split
partials (M-LRD length-aware plan) and grouped-latent scores and partials live in the library's static
per-GPU scratch array instead of a caller workspace. Its output must equal palu_sdpa_decode's (with a
workspace) on the same inputs, bit for bit in deterministic mode, on two calls in a row, the second with a
smaller input; both are also held to the oracle bar (max-abs 2e-2, cosine 0.9999). Shapes whose scratch
need exceeds the array are rejected before any launch.
"""
import ctypes

import pytest
import torch

from oracle import palu_oracle as ref
from palu_tt import _native, fused
from palu_tt.cache import GroupedLatentCache, LatentCache

HD = 128
THETA = 500000.0
LLAMA3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}


def _case(dev, B, S, r_k, r_v, nh, nkv, n_groups, seed):
    g = torch.Generator().manual_seed(seed)
    bf = lambda *s, std=1.0: (torch.randn(*s, generator=g) * std).to(torch.bfloat16)
    c = {"q": bf(1, B, nh, HD), "k": bf(B, n_groups, S, r_k), "v": bf(B, n_groups, S, r_v),
         "u_k": bf(nkv, r_k, HD, std=r_k ** -0.5), "u_v": bf(nkv, r_v, HD, std=r_v ** -0.5) if n_groups < nkv else None,
         "pos": torch.randint(0, S, (B,), generator=g)}
    c["pos"][0] = S - 1
    cos, sin = fused.cos_sin_tables(HD, S, THETA, LLAMA3)
    c["cos"], c["sin"] = cos, sin
    d = {"q": c["q"].to(dev), "k": LatentCache.from_rows(c["k"].to(dev), "k").data,
         "v": LatentCache.from_rows(c["v"].to(dev), "v").data,
         "w_rot": fused.w_rot_from_u_k(c["u_k"].float()).to(dev, torch.bfloat16).contiguous(),
         "cs": fused.cs_table(cos, sin, S).to(dev).contiguous(), "pos": c["pos"].to(dev, torch.int32),
         "u_v": None if c["u_v"] is None else c["u_v"].to(dev).contiguous()}
    dims = dict(B=B, S=S, r_k=r_k, r_v=r_v, nh=nh, nkv=nkv, n_groups=n_groups, dv=HD if c["u_v"] is not None else r_v)
    return c, d, dims


def _call(lib, d, dims, noalloc):
    dev = d["q"].device
    out = torch.full((1, dims["B"], dims["nh"], dims["dv"]), float("nan"), dtype=torch.float32, device=dev)
    common = [_native.ptr(d["q"]), _native.ptr(d["k"]), _native.ptr(d["w_rot"]), _native.ptr(d["cs"]),
              _native.ptr(d["v"]), dims["dv"], _native.ptr(d["pos"]), _native.ptr(out), None, None,
              _native.ptr(d["u_v"]), None, HD ** -0.5, 0, 2, 1, 0, dims["B"], dims["nh"], dims["nkv"], dims["n_groups"],
              dims["S"], dims["r_k"], dims["r_v"], 2 * HD, dims["S"], 2 * HD, _native.DTYPE_F32, _native.DTYPE_F32,
              _native.LAYOUT_TILED, 1]
    stream = _native.stream_handle(dev)
    if noalloc:
        rc = lib.palu_sdpa_decode_noalloc(*common, stream)
    else:
        if d["u_v"] is not None:
            need = lib.palu_glrd_workspace_bytes(dims["B"], dims["nh"], dims["nkv"], dims["n_groups"], dims["S"], dims["r_v"])
        else:
            need = lib.palu_decode_workspace_bytes(dims["B"], dims["nkv"], dims["S"], dims["dv"])
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        rc = lib.palu_sdpa_decode(*common, _native.ptr(ws), need, stream)
    _native.check(rc)
    torch.cuda.synchronize()
    return out.cpu()


def _oracle(c):
    return ref.reference_decode(c["q"].float(), c["k"].float(), c["u_k"].float(), c["v"].float(), c["pos"],
                                c["cos"], c["sin"], HD ** -0.5, u_v=None if c["u_v"] is None else c["u_v"].float())


@pytest.mark.gpu
@pytest.mark.parametrize("shapes", [
    # M-LRD: 40 and 24 items, both cut into length-aware chunks merged through the scratch
    [dict(B=5, S=1024, r_k=64, r_v=64, nh=32, nkv=8, n_groups=8), dict(B=3, S=512, r_k=64, r_v=64, nh=32, nkv=8, n_groups=8)],
    # G-LRD: scores and PV partials in the scratch
    [dict(B=2, S=2048, r_k=256, r_v=256, nh=32, nkv=8, n_groups=2), dict(B=1, S=1024, r_k=128, r_v=192, nh=32, nkv=8, n_groups=2)],
])
def test_noalloc_equals_the_workspace_entry_point(gpu, shapes):
    lib = _native.load()
    for i, sh in enumerate(shapes):
        c, d, dims = _case(gpu, seed=100 + i, **sh)
        with_ws = _call(lib, d, dims, noalloc=False)
        no_alloc = _call(lib, d, dims, noalloc=True)
        assert torch.equal(no_alloc, with_ws), f"call {i}: max diff {(no_alloc - with_ws).abs().max():.3e}"
        exp = _oracle(c)
        ma, cs = ref.max_abs(no_alloc, exp), ref.cosine(no_alloc, exp)
        assert ma <= 2e-2 and cs >= 0.9999, f"call {i}: max_abs {ma:.3e}, cosine {cs:.6f}"


def _layouts_case(dev, kind, B, S, seed, ranks=None):
    """Inputs for one call of the layout cases: 'grouped' -- compact GroupedLatentCaches of unequal group
    ranks (PALU_LAYOUT_TILED_GROUPED with the groups' ranks); 'rows_glrd' -- the reference's row-major
    grouped latents; 'tiled_rows' -- M-LRD with the output in the tiled activation layout
    (PALU_OUT_TILED_ROWS)."""
    g = torch.Generator().manual_seed(seed)
    bf = lambda *s, std=1.0: (torch.randn(*s, generator=g) * std).to(torch.bfloat16)
    nh, nkv = 32, 8
    cos, sin = fused.cos_sin_tables(HD, S, THETA, LLAMA3)
    pos = torch.randint(0, S, (B,), generator=g)
    pos[0] = S - 1
    kw = dict(scale=HD ** -0.5, deterministic=True)
    if kind == "tiled_rows":
        r = 64
        k, v = bf(B, nkv, S, r).to(dev), bf(B, nkv, S, r).to(dev)
        u_k = bf(nkv, r, HD, std=r ** -0.5)
        args = (bf(1, B, nh, HD).to(dev), LatentCache.from_rows(k, "k"),
                fused.w_rot_from_u_k(u_k.float()).to(dev, torch.bfloat16)[None],
                fused.cs_table(cos, sin, S)[None, None].to(dev), LatentCache.from_rows(v, "v"), r,
                pos.to(dev, torch.int32))
        return args, dict(kw, tiled_rows=True), lambda: torch.zeros(64, nh * r, dtype=torch.bfloat16, device=dev)
    rk, rv = ranks
    ng = 2
    k, v = bf(B, ng, S, max(rk)), bf(B, ng, S, max(rv))
    u_k, u_v = bf(nkv, max(rk), HD, std=0.08), bf(nkv, max(rv), HD, std=0.08)
    for gi in range(ng):
        k[:, gi, :, rk[gi]:] = 0
        v[:, gi, :, rv[gi]:] = 0
        u_k[4 * gi:4 * gi + 4, rk[gi]:] = 0
        u_v[4 * gi:4 * gi + 4, rv[gi]:] = 0
    if kind == "grouped":
        kc, vc = GroupedLatentCache.from_rows(k.to(dev), rk, "k"), GroupedLatentCache.from_rows(v.to(dev), rv, "v")
    else:
        kc, vc = k.to(dev), v.to(dev)
    args = (bf(1, B, nh, HD).to(dev), kc, fused.w_rot_from_u_k(u_k.float()).to(dev, torch.bfloat16)[None],
            fused.cs_table(cos, sin, S)[None, None].to(dev), vc, HD, pos.to(dev, torch.int32))
    return args, dict(kw, u_v=u_v.to(dev)[None], group_ranks=(rk, rv), out_dtype=torch.float32), \
        lambda: torch.zeros(1, B, nh, HD, dtype=torch.float32, device=dev)


@pytest.mark.gpu
@pytest.mark.parametrize("kind,calls", [
    ("grouped", [(2, 2048, ([96, 192], [256, 64])), (1, 1024, ([64, 128], [128, 32]))]),
    ("rows_glrd", [(2, 1000, ([128, 256], [192, 96])), (1, 512, ([32, 64], [64, 64]))]),
    ("tiled_rows", [(16, 1024, None), (8, 512, None)]),
])
def test_noalloc_equals_the_workspace_entry_point_on_other_layouts(gpu, kind, calls):
    """palu_sdpa_decode_noalloc sets its own strides and scratch for every layout: compact grouped caches
    of unequal group ranks, the reference's row-major grouped latents (S = 1000, not a multiple of the
    32-position block), and the tiled-rows output the decode step's output projection reads. Each is
    compared bit for bit with palu_sdpa_decode (workspace) on two calls in a row, the second smaller."""
    for i, (B, S, ranks) in enumerate(calls):
        args, kw, fresh = _layouts_case(gpu, kind, B, S, seed=300 + i, ranks=ranks)
        with_ws = fused.palu_sdpa_decode(*args, out=fresh(), **kw)
        no_alloc = fused.palu_sdpa_decode(*args, out=fresh(), noalloc=True, **kw)
        torch.cuda.synchronize()
        assert torch.isfinite(with_ws.float()).all()
        assert torch.equal(no_alloc.cpu(), with_ws.cpu()), \
            f"{kind} call {i}: max diff {(no_alloc.float() - with_ws.float()).abs().max():.3e}"


def test_noalloc_rejects_shapes_beyond_the_scratch():
    """Checked before the device is touched, so it runs without a GPU too."""
    lib = _native.load()
    fake = ctypes.c_void_p(1 << 20)
    B, S, nq, nkv, G, r = 64, 65536, 32, 8, 2, 512          # grouped-latent scores alone: 512 MiB
    assert lib.palu_glrd_workspace_bytes(B, nq, nkv, G, S, r) > _native.NOALLOC_SCRATCH_BYTES
    rc = lib.palu_sdpa_decode_noalloc(fake, fake, fake, fake, fake, HD, fake, fake, None, None, fake, None, 0.088, 0, 2, 1,
                                      0, B, nq, nkv, G, S, r, r, 2 * HD, S, 2 * HD, 0, 1, _native.LAYOUT_TILED, 0,
                                      None)
    assert rc == _native.PALU_EUNSUPPORTED and "scratch" in lib.palu_last_error().decode()
