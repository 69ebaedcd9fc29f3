"""GPU parity of the paged latent cache: paged fused decode, paged stock decode and paged append.

The oracle gathers the pages of every row into contiguous rows (oracle.gather_pages) and runs the same
fp32 decode; the bar is the decode bar (max-abs 2e-2, cosine 0.9999). Page pools are filled from
contiguous rows through a random permutation of pages, rows have ragged lengths (positions in the
middle of a page and of a 32-position block), and the mixed-rank shapes (r_k, r_v) = (32, 128) and
(128, 64) with 64-token pages and lengths up to 32768 cover the paged configuration of the hot path.
"""
import pytest
import torch

from oracle import palu_oracle as ref
from palu_tt import fused
from palu_tt.cache import LatentCache

pytestmark = pytest.mark.gpu

HD = 128
THETA = 500000.0
LLAMA3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}


def _bf(t):
    return t.to(torch.bfloat16).float()


def _paged(rows, page_size, g, spare=3):
    """Scatter contiguous rows [B, G, S, r] into a pool through a random page permutation; returns
    (pool [n_pages, G, page_size, r], page_table [B, S / page_size] int32)."""
    B, G, S, r = rows.shape
    mp = S // page_size
    n_pages = B * mp + spare
    perm = torch.randperm(n_pages, generator=g)[:B * mp].view(B, mp).to(torch.int32)
    pool = torch.randn(n_pages, G, page_size, r, generator=g)          # unused pages hold noise
    for b in range(B):
        for j in range(mp):
            pool[perm[b, j]] = rows[b, :, j * page_size:(j + 1) * page_size]
    return pool, perm


def _case(B, S, r_k, r_v, page_size, seed, nh=32, nkv=8, lengths=None):
    g = torch.Generator().manual_seed(seed)
    q = _bf(torch.randn(1, B, nh, HD, generator=g))
    k = _bf(torch.randn(B, nkv, S, r_k, generator=g))
    v = _bf(torch.randn(B, nkv, S, r_v, generator=g))
    u_k = _bf(torch.randn(nkv, r_k, HD, generator=g) / r_k ** 0.5)
    if lengths is None:
        pos = torch.randint(0, S, (B,), generator=g)
        pos[0] = S - 1
        if B > 2:
            pos[1], pos[2] = page_size - 1 + page_size // 2, 40
    else:
        pos = torch.tensor(lengths) - 1
    kp, pt = _paged(k, page_size, g)
    vp = torch.randn(kp.shape[0], nkv, page_size, r_v, generator=g)     # V pages on K's page table
    for b in range(B):
        for j in range(S // page_size):
            vp[pt[b, j]] = v[b, :, j * page_size:(j + 1) * page_size]
    return q, k, v, u_k, pos, _bf(kp), _bf(vp), pt


def _decode(dev, q, kp, vp, u_k, pos, pt, S, layout, **kw):
    cos, sin = fused.cos_sin_tables(HD, S, THETA, LLAMA3)
    kd, vd = kp.to(dev, torch.bfloat16), vp.to(dev, torch.bfloat16)
    if layout == "tiled":
        kd, vd = LatentCache.from_rows(kd, "k"), LatentCache.from_rows(vd, "v")
    out = fused.palu_sdpa_decode(q.to(dev, torch.bfloat16), kd, fused.w_rot_from_u_k(u_k).to(dev, torch.bfloat16)[None],
                                 fused.cs_table(cos, sin, S)[None, None].to(dev), vd, vp.shape[-1],
                                 pos.to(dev, torch.int32), scale=HD ** -0.5, out_dtype=torch.float32,
                                 page_table_tensor=pt.to(dev), **kw)
    torch.cuda.synchronize()
    return out.cpu()


def _check(out, exp):
    ma, cs = ref.max_abs(out, exp), ref.cosine(out, exp)
    assert torch.isfinite(out).all() and ma <= 2e-2 and cs >= 0.9999, f"max_abs {ma:.3e}, cosine {cs:.6f}"


_WIDTHS_32 = [(64, 64, 64), (32, 128, 64), (128, 64, 64), (64, 32, 32), (96, 96, 128)]
_WIDTHS_16 = [(64, 80, 64), (80, 64, 64), (48, 112, 32)]      # tiled caches only: 16-wide V tiles, K half tiles


@pytest.mark.parametrize("layout,r_k,r_v,page_size", [(lay, *w) for lay in ("rows", "tiled") for w in _WIDTHS_32] +
                         [("tiled", *w) for w in _WIDTHS_16])
def test_paged_decode_matches_oracle(gpu, layout, r_k, r_v, page_size):
    B, S = 4, 2048
    q, k, v, u_k, pos, kp, vp, pt = _case(B, S, r_k, r_v, page_size, seed=r_k + r_v + page_size)
    assert torch.equal(ref.gather_pages(kp, pt), k) and torch.equal(ref.gather_pages(vp, pt), v)
    cos, sin = ref.cos_sin_tables(HD, S, THETA, LLAMA3)
    exp = ref.reference_decode(q, k, u_k, v, pos, cos, sin, HD ** -0.5)
    _check(_decode(gpu, q, kp, vp, u_k, pos, pt, S, layout), exp)


@pytest.mark.parametrize("layout", ["rows", "tiled"])
def test_paged_equals_contiguous_bit_for_bit(gpu, layout):
    """Same rows, same split plan, fixed block order: the paged kernel must reproduce the contiguous one."""
    B, S = 3, 1024
    q, k, v, u_k, pos, kp, vp, pt = _case(B, S, 64, 64, 64, seed=7)
    paged = _decode(gpu, q, kp, vp, u_k, pos, pt, S, layout, deterministic=True)
    cos, sin = fused.cos_sin_tables(HD, S, THETA, LLAMA3)
    kd, vd = k.to(gpu, torch.bfloat16), v.to(gpu, torch.bfloat16)
    if layout == "tiled":
        kd, vd = LatentCache.from_rows(kd, "k"), LatentCache.from_rows(vd, "v")
    contig = fused.palu_sdpa_decode(q.to(gpu, torch.bfloat16), kd, fused.w_rot_from_u_k(u_k).to(gpu, torch.bfloat16)[None],
                                    fused.cs_table(cos, sin, S)[None, None].to(gpu), vd, 64, pos.to(gpu, torch.int32),
                                    scale=HD ** -0.5, out_dtype=torch.float32, deterministic=True).cpu()
    assert torch.equal(paged, contig)


@pytest.mark.parametrize("r_k,r_v", [(32, 128), (128, 64)])
def test_paged_mixed_ranks_long_ragged_rows(gpu, r_k, r_v):
    """B=8 rows with lengths drawn from U[1024, 32768], 64-token pages."""
    B, S, ps = 8, 32768, 64
    g = torch.Generator().manual_seed(31 + r_k)
    lengths = torch.randint(1024, S + 1, (B,), generator=g).tolist()
    lengths[0] = S
    q, k, v, u_k, pos, kp, vp, pt = _case(B, S, r_k, r_v, ps, seed=r_k, lengths=lengths)
    cos, sin = ref.cos_sin_tables(HD, S, THETA, LLAMA3)
    exp = ref.reference_decode(q, k, u_k, v, pos, cos, sin, HD ** -0.5)
    _check(_decode(gpu, q, kp, vp, u_k, pos, pt, S, "tiled"), exp)


def test_paged_skewed_rows_more_items_than_one_fill(gpu):
    """Length-aware chunk plan over pages: 34 rows x 8 KV heads (272 items: 512 workgroups), lengths from
    one token to the whole cache, 64-token pages in a shuffled pool."""
    B, S, ps = 34, 512, 64
    g = torch.Generator().manual_seed(77)
    lengths = torch.randint(1, S + 1, (B,), generator=g).tolist()
    lengths[0], lengths[1], lengths[2] = S, 1, 33
    q, k, v, u_k, pos, kp, vp, pt = _case(B, S, 64, 64, ps, seed=5, lengths=lengths)
    cos, sin = ref.cos_sin_tables(HD, S, THETA, LLAMA3)
    exp = ref.reference_decode(q, k, u_k, v, pos, cos, sin, HD ** -0.5)
    _check(_decode(gpu, q, kp, vp, u_k, pos, pt, S, "tiled"), exp)


@pytest.mark.parametrize("layout", ["rows", "tiled"])
def test_paged_append_then_decode(gpu, layout):
    """Append one new latent row per sequence through the page table, then decode at that position."""
    B, S, ps, r = 4, 512, 64, 64
    q, k, v, u_k, pos, kp, vp, pt = _case(B, S, r, r, ps, seed=3)
    g = torch.Generator().manual_seed(5)
    new_pos = torch.tensor([S - 1, 63, 64, 300])
    new_k = _bf(torch.randn(B, 8, r, generator=g))
    new_v = _bf(torch.randn(B, 8, r, generator=g))
    kd, vd = kp.to(gpu, torch.bfloat16), vp.to(gpu, torch.bfloat16)
    if layout == "tiled":
        kd, vd = LatentCache.from_rows(kd, "k"), LatentCache.from_rows(vd, "v")
    ptd = pt.to(gpu)
    fused.paged_update_cache(kd, new_k.to(gpu, torch.bfloat16), new_pos.to(gpu, torch.int32), page_table=ptd)
    fused.paged_update_cache(vd, new_v.to(gpu, torch.bfloat16), new_pos.to(gpu, torch.int32), page_table=ptd)
    torch.cuda.synchronize()
    kr = (kd.to_rows() if layout == "tiled" else kd).float().cpu()
    vr = (vd.to_rows() if layout == "tiled" else vd).float().cpu()
    k2, v2 = k.clone(), v.clone()
    for b in range(B):
        k2[b, :, new_pos[b]] = new_k[b]
        v2[b, :, new_pos[b]] = new_v[b]
    assert torch.equal(ref.gather_pages(kr, pt), k2) and torch.equal(ref.gather_pages(vr, pt), v2)
    # pages no row maps to are untouched
    used = set(pt.flatten().tolist())
    for p_ in range(kp.shape[0]):
        if p_ not in used:
            assert torch.equal(kr[p_], kp[p_])
    cos, sin = ref.cos_sin_tables(HD, S, THETA, LLAMA3)
    exp = ref.reference_decode(q, k2, u_k, v2, new_pos, cos, sin, HD ** -0.5)
    cs = fused.cos_sin_tables(HD, S, THETA, LLAMA3)
    out = fused.palu_sdpa_decode(q.to(gpu, torch.bfloat16), kd, fused.w_rot_from_u_k(u_k).to(gpu, torch.bfloat16)[None],
                                 fused.cs_table(*cs, S)[None, None].to(gpu), vd, r, new_pos.to(gpu, torch.int32),
                                 scale=HD ** -0.5, out_dtype=torch.float32, page_table_tensor=ptd)
    torch.cuda.synchronize()
    _check(out.cpu(), exp)


@pytest.mark.parametrize("layout", ["rows", "tiled"])
def test_paged_stock_decode_matches_full_kv_oracle(gpu, layout):
    B, S, ps, nkv, dv = 4, 1024, 64, 8, 128
    g = torch.Generator().manual_seed(11)
    q = _bf(torch.randn(1, B, 32, HD, generator=g))
    k = _bf(torch.randn(B, nkv, S, HD, generator=g))
    v = _bf(torch.randn(B, nkv, S, dv, generator=g))
    kp, pt = _paged(k, ps, g)
    vp = torch.zeros(kp.shape[0], nkv, ps, dv)
    for b in range(B):
        for j in range(S // ps):
            vp[pt[b, j]] = v[b, :, j * ps:(j + 1) * ps]
    pos = torch.tensor([S - 1, 0, 100, 777])
    exp = ref.full_kv_decode(q, k, v, pos, HD ** -0.5)
    kd, vd = kp.to(gpu, torch.bfloat16), _bf(vp).to(gpu, torch.bfloat16)
    if layout == "tiled":
        kd, vd = LatentCache.from_rows(kd, "k"), LatentCache.from_rows(vd, "v")
    out = fused.flash_decode(q.to(gpu, torch.bfloat16), kd, vd, pos.to(gpu, torch.int32), scale=HD ** -0.5,
                             out_dtype=torch.float32, page_table_tensor=pt.to(gpu))
    torch.cuda.synchronize()
    _check(out.cpu(), exp)


def test_split_items_repeat_exactly_on_one_shared_workspace(gpu):
    """Split items (8 rows x 8 KV heads on a 256-workgroup plan) merge inside the decode launch: each
    chunk counts itself into an 8-byte counter of its item in the workspace, and the chunk that completes
    the count merges the item. Two inputs alternate on one workspace that first holds stale counter words
    (the fixed tag with a call number no launch carries and a nonzero count), with a call of other widths in between
    whose partial slots overlay these calls' counters: every output must equal its input's first output
    bit for bit, and match the oracle."""
    S, ps = 8192, 64
    cases = []
    for seed, r_k, r_v in ((1, 64, 64), (2, 64, 64), (3, 32, 128)):
        g = torch.Generator().manual_seed(100 + seed)
        lengths = torch.randint(1, S + 1, (8,), generator=g).tolist()
        lengths[0] = S
        cases.append(_case(8, S, r_k, r_v, ps, seed=seed, lengths=lengths))
    from palu_tt import _native
    need = max(_native.load().palu_decode_workspace_bytes(8, 8, S, c[2].shape[-1]) for c in cases)
    assert need > 0, "the plan must split items for this test"
    ws = torch.empty(need // 8 + 1, dtype=torch.int64, device=gpu)
    stale = (0xA5C3 << 48) | (0 << 16) | 5                 # call number 0 (no launch's), five chunks counted
    ws.fill_(stale - (1 << 64))
    cos, sin = ref.cos_sin_tables(HD, S, THETA, LLAMA3)
    first = {}
    for it, i in enumerate([0, 1, 0, 2, 1, 0, 2, 1, 1, 0, 0]):
        q, k, v, u_k, pos, kp, vp, pt = cases[i]
        out = _decode(gpu, q, kp, vp, u_k, pos, pt, S, "tiled", workspace=ws)
        if i not in first:
            first[i] = out
            _check(out, ref.reference_decode(q, k, u_k, v, pos, cos, sin, HD ** -0.5))
        else:
            assert torch.equal(out, first[i]), f"call {it} (input {i}) differs from that input's first call"
