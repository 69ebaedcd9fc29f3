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
                                                   ("tiled", "k", 4, 384), ("tiled", "v", 2, 256), ("rows", "v", 4, 512),
                                                   ("tiled", "k", 1, 112)])
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


def _linear_ref(x, w):
    return x.float() @ w.float().T


def _check_linear(y, ref):
    y = y.float()
    scale = ref.abs().max().item()
    err = (y - ref).abs().max().item()
    cos = F.cosine_similarity(y.flatten(), ref.flatten(), dim=0).item()
    # bf16 output of an fp32 sum: one rounding of the result (2^-8 relative) plus summation order
    assert err <= scale * 2 ** -7 and cos >= 0.99999, f"max-abs {err:.3e} of scale {scale:.3e}, cosine {cos:.7f}"


@pytest.mark.parametrize("rows,n,k", [(64, 4096, 4096), (64, 5120, 4096), (64, 4096, 2432), (64, 28672, 4096),
                                      (64, 4096, 14336), (17, 6144, 4096), (1, 256, 1024), (5, 48, 96)])
def test_linear_tiled_matches_fp32(gpu, rows, n, k):
    """The decode projections at the 32-layer decoder's shapes (QKV, output, gate/up, down) and small,
    ragged ones, with the plan's work split, against fp32 torch on the same bf16 inputs."""
    g = torch.Generator().manual_seed(n + k + rows)
    x = torch.randn(rows, k, generator=g).to(gpu, torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.02).to(gpu, torch.bfloat16)
    rtw, ks = decoder_ops.linear_plan(rows, n, k)
    y = decoder_ops.linear_tiled(x, decoder_ops.tile_weight(w, rtw), rtw, ks)
    torch.cuda.synchronize()
    _check_linear(y, _linear_ref(x, w))


@pytest.mark.parametrize("rtw,ks", [(1, 1), (2, 4), (3, 2), (5, 1), (7, 8), (8, 3), (8, 16), (4, 64)])
def test_linear_tiled_every_work_split(gpu, rtw, ks):
    """Every row-tile grouping and k-slice count, including ones that leave the last group short (n = 400:
    25 row tiles), slices with an odd step count per wave, and more slices than k tiles can fill."""
    g = torch.Generator().manual_seed(rtw * 100 + ks)
    x = torch.randn(40, 1344, generator=g).to(gpu, torch.bfloat16)
    w = (torch.randn(400, 1344, generator=g) * 0.05).to(gpu, torch.bfloat16)
    y = decoder_ops.linear_tiled(x, decoder_ops.tile_weight(w, rtw), rtw, ks)
    torch.cuda.synchronize()
    _check_linear(y, _linear_ref(x, w))


def test_linear_tiled_strided_views_and_repeat(gpu):
    """x and out as column slices of wider rows (the QKV output layout), a caller workspace, and a
    bit-identical repeat (the k-slice sums and the wave tree run in a fixed order)."""
    g = torch.Generator().manual_seed(11)
    xw = torch.randn(64, 4096 + 64, generator=g).to(gpu, torch.bfloat16)
    x = xw[:, 32:32 + 4096]
    w = (torch.randn(1024, 4096, generator=g) * 0.02).to(gpu, torch.bfloat16)
    wt = decoder_ops.tile_weight(w, 2)
    ow = torch.zeros(64, 1024 + 16, dtype=torch.bfloat16, device=gpu)
    out = ow[:, 8:8 + 1024]
    ws = torch.empty(4 * 64 * 1024 * 4, dtype=torch.uint8, device=gpu)
    decoder_ops.linear_tiled(x, wt, 2, 4, out=out, workspace=ws)
    again = decoder_ops.linear_tiled(x, wt, 2, 4)
    torch.cuda.synchronize()
    _check_linear(out, _linear_ref(x, w))
    assert torch.equal(out, again)
    assert (ow[:, :8] == 0).all() and (ow[:, 8 + 1024:] == 0).all()


def test_linear_tiled_rejects_bad_shapes(gpu):
    x = torch.zeros(65, 64, dtype=torch.bfloat16, device=gpu)
    wt = torch.zeros(32, 64, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="1..64"):
        decoder_ops.linear_tiled(x, wt, 1, 1)
    with pytest.raises(RuntimeError, match="multiple of 16"):
        decoder_ops.linear_tiled(x[:8], torch.zeros(24, 64, dtype=torch.bfloat16, device=gpu), 1, 1)
    with pytest.raises(RuntimeError, match="rtw"):
        decoder_ops.linear_tiled(x[:8], wt, 9, 1)


@pytest.mark.parametrize("rows,n,k,rtw,ks", [(64, 28672, 4096, 7, 1), (64, 4096, 14336, 4, 4), (23, 4096, 2432, 1, 1),
                                             (64, 400, 1344, 3, 2)])
def test_linear_tiled_activations(gpu, rows, n, k, rtw, ks):
    """Activations in the 64-row tiled layout (tile_rows) give the same result as row-major ones, bit for
    bit (same products, same order), and match fp32; the pad rows past the live count hold NaN and are
    ignored."""
    g = torch.Generator().manual_seed(rows * 7 + rtw)
    x = torch.randn(rows, k, generator=g).to(gpu, torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.02).to(gpu, torch.bfloat16)
    wt = decoder_ops.tile_weight(w, rtw)
    padded = torch.full((64, k), float("nan"), dtype=torch.bfloat16, device=gpu)
    padded[:rows] = x
    xt = decoder_ops.tile_weight(padded, 4)
    a = decoder_ops.linear_tiled(xt, wt, rtw, ks, x_tiled=True, rows=rows)
    b = decoder_ops.linear_tiled(x, wt, rtw, ks)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    _check_linear(a, _linear_ref(x, w))


def _argmax_case(gpu, rows, n, k, rtw, x_tiled, seed, plant=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, k, generator=g)
    w = torch.randn(n, k, generator=g) * 0.05
    if plant:
        plant(x, w)
    x, w = x.to(gpu, torch.bfloat16), w.to(gpu, torch.bfloat16)
    wt = decoder_ops.tile_weight(w, rtw)
    if x_tiled:
        padded = torch.zeros(64, k, dtype=torch.bfloat16, device=gpu)
        padded[:rows] = x
        xa, kw = decoder_ops.tile_weight(padded, 4), dict(x_tiled=True, rows=rows)
    else:
        xa, kw = x, {}
    ids = decoder_ops.linear_argmax(xa, wt, rtw, **kw)
    logits = decoder_ops.linear_tiled(xa, wt, rtw, 1, **kw)
    want = decoder_ops.argmax_rows(logits)
    torch.cuda.synchronize()
    return ids, want, logits


@pytest.mark.parametrize("rows,n,k,rtw,x_tiled", [(64, 128256, 256, 8, True), (9, 128256, 256, 8, False),
                                                   (64, 4800, 1344, 1, True), (33, 16016, 96, 3, False),
                                                   (64, 16 * 2053, 160, 8, True), (1, 256, 1024, 2, False),
                                                   (64, 4096, 4096, 8, True)])
def test_linear_argmax_matches_argmax_of_the_logits(gpu, rows, n, k, rtw, x_tiled):
    """The fused LM-head pick equals argmax_rows of linear_tiled's bf16 logits (ks = 1) id for id, and
    torch.argmax of those logits: the LM head's 1,002 groups of 8 row tiles and fewer groups than
    workgroups, ragged last groups, short rows, k tiles fewer than the waves, row-major and tiled x."""
    ids, want, logits = _argmax_case(gpu, rows, n, k, rtw, x_tiled, seed=n + rows + rtw)
    assert ids.dtype == torch.int64 and ids.shape == (rows,)
    assert torch.equal(ids, want)
    assert torch.equal(ids.cpu(), torch.argmax(logits.float().cpu(), dim=-1))


def test_linear_argmax_ties_nan_and_zeros(gpu):
    """Equal maxima pick the first column, within a group of row tiles and across groups (duplicated
    weight rows give bit-identical logits); a NaN column wins over every number, the first of two; an
    all-zero activation row gives all-zero logits and id 0; torch.argmax agrees on every row."""
    n, k = 16 * 700, 256

    def plant(x, w):
        w[3000] = w[100] * 4                                  # row 0's maximum, twice: 100 first
        w[2000] = w[100] * 4
        w[100] = w[100] * 4
        w[17] = w[9]                                          # the same group of 8 row tiles
        x[0] = w[100] / w[100].norm()
        x[1] = w[9] / w[9].norm()
        x[2].zero_()
        w[5000, 7] = float("nan")                            # NaN columns 5000 and 9000: 5000 wins
        w[9000, 3] = float("nan")

    ids, want, logits = _argmax_case(gpu, 16, n, k, 8, True, seed=5, plant=plant)
    assert torch.equal(ids, want)
    assert torch.equal(ids.cpu(), torch.argmax(logits.float().cpu(), dim=-1))
    assert ids[0].item() == 5000 and ids[2].item() == 5000          # NaN above every number
    lg = logits.float().cpu()
    lg[:, 5000] = lg[:, 9000] = float("-inf")
    assert torch.argmax(lg[0]).item() == 100 and torch.argmax(lg[1]).item() == 9


def test_linear_argmax_without_nan_ties(gpu):
    """The same planted ties without NaN columns: row 0 picks column 100 of three equal maxima (the
    others 1,900 and 2,900 columns later, other groups), row 1 column 9 of two (9 and 17, one group),
    the all-zero row column 0."""
    n, k = 16 * 700, 256

    def plant(x, w):
        w[100] = w[100] * 4
        w[2000] = w[100]
        w[3000] = w[100]
        w[17] = w[9]
        x[0] = w[100] / w[100].norm()
        x[1] = w[9] / w[9].norm()
        x[2].zero_()

    ids, want, logits = _argmax_case(gpu, 16, n, k, 8, False, seed=6, plant=plant)
    assert torch.equal(ids, want)
    assert ids[0].item() == 100 and ids[1].item() == 9 and ids[2].item() == 0
    assert torch.equal(ids.cpu(), torch.argmax(logits.float().cpu(), dim=-1))


def test_linear_argmax_rejects_bad_arguments(gpu):
    x = torch.zeros(8, 64, dtype=torch.bfloat16, device=gpu)
    wt = torch.zeros(32, 64, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="workspace"):
        decoder_ops.linear_argmax(x, wt, 1, workspace=torch.empty(16, dtype=torch.uint8, device=gpu))
    with pytest.raises(RuntimeError, match="rtw"):
        decoder_ops.linear_argmax(x, wt, 9)


@pytest.mark.parametrize("rows,n,stride", [(64, 128256, 128256), (3, 1000, 1008), (1, 7, 8), (5, 4099, 4104)])
def test_argmax_rows_matches_torch(gpu, rows, n, stride):
    """First index among equal maxima (planted ties, a row of equal values), NaN above every number."""
    g = torch.Generator().manual_seed(n)
    buf = torch.randn(rows, stride, generator=g).to(torch.bfloat16)
    x = buf[:, :n]
    x[0, n // 3] = x[0, n - 1] = 9.0                        # tie: the first index wins
    if rows > 1:
        x[1] = 0.5                                           # all equal: index 0
    if rows > 2:
        x[2, n // 2] = float("nan")                          # NaN wins over every number
        x[2, n - 2] = float("nan")
    xd = buf.to(gpu)[:, :n]
    got = decoder_ops.argmax_rows(xd)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), torch.argmax(x.float(), dim=-1))


@pytest.mark.parametrize("rows", [64, 9])
def test_rmsnorm_and_swiglu_write_the_tiled_layout(gpu, rows):
    """rmsnorm / swiglu with tiled_out write exactly tile_rows of their row-major outputs."""
    g = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, 4096, generator=g).to(gpu, torch.bfloat16)
    w = (1 + 0.1 * torch.randn(4096, generator=g)).to(gpu, torch.bfloat16)
    gu = torch.randn(rows, 2 * 1024, generator=g).to(gpu, torch.bfloat16)
    y = decoder_ops.rmsnorm(x, w, 1e-5)
    yt = torch.zeros(64, 4096, dtype=torch.bfloat16, device=gpu)
    decoder_ops.rmsnorm(x, w, 1e-5, out=yt, tiled_out=True)
    s = decoder_ops.swiglu(gu)
    st = torch.zeros(64, 1024, dtype=torch.bfloat16, device=gpu)
    decoder_ops.swiglu(gu, out=st, tiled_out=True)
    torch.cuda.synchronize()
    assert torch.equal(yt, decoder_ops.tile_rows(y))
    assert torch.equal(st, decoder_ops.tile_rows(s))
    with pytest.raises(RuntimeError, match="tiled output"):
        decoder_ops.rmsnorm(torch.zeros(65, 64, dtype=torch.bfloat16, device=gpu), w[:64], 1e-5,
                            out=torch.zeros(64, 64, dtype=torch.bfloat16, device=gpu), tiled_out=True)


@pytest.mark.parametrize("rtw,ks", [(4, 4), (3, 2), (7, 1)])
def test_linear_partials_mode(gpu, rtw, ks):
    """mode="partials" returns the k slices' fp32 sums; added up in slice order they are what the bf16
    mode rounds (bit for bit once rounded), and they match fp32."""
    g = torch.Generator().manual_seed(rtw * 10 + ks)
    x = torch.randn(64, 2048, generator=g).to(gpu, torch.bfloat16)
    w = (torch.randn(1024, 2048, generator=g) * 0.02).to(gpu, torch.bfloat16)
    wt = decoder_ops.tile_weight(w, rtw)
    part = decoder_ops.linear_tiled(x, wt, rtw, ks, mode="partials")
    y = decoder_ops.linear_tiled(x, wt, rtw, ks)
    torch.cuda.synchronize()
    assert part.shape == (ks, 64, 1024) and part.dtype == torch.float32
    s = part[0].clone()
    for k in range(1, ks):
        s += part[k]
    assert torch.equal(s.to(torch.bfloat16), y)
    _check_linear(s, _linear_ref(x, w))


@pytest.mark.parametrize("rows,x_tiled,rtw", [(64, True, 0), (64, False, 0), (13, True, 0), (64, True, 7), (29, True, 8),
                                              (64, True, 1), (64, True, 3)])
def test_linear_swiglu_mode(gpu, rows, x_tiled, rtw):
    """The gate / up projection with SwiGLU in its epilogue (interleave_gate_up weight, tiled output)
    equals silu(x w_gate^T) * (x w_up^T) from fp32 products, one bf16 rounding at the end. Explicit row
    tiles per workgroup: each wave's tiles are stored in pairs, so 7 and 3 (an odd count per wave, 192
    row tiles leaving a short last group for 7) and 1 (one unpaired tile) cover the unpaired ends."""
    g = torch.Generator().manual_seed(rows + x_tiled + 100 * rtw)
    k, f = 1024, 1536
    x = torch.randn(rows, k, generator=g).to(gpu, torch.bfloat16)
    wg = (torch.randn(f, k, generator=g) * 0.05).to(gpu, torch.bfloat16)
    wu = (torch.randn(f, k, generator=g) * 0.05).to(gpu, torch.bfloat16)
    lin = decoder_ops.DecodeLinear(None, 64, gate_up=(wg, wu), rtw=rtw, ks=1 if rtw else 0)
    assert lin.tiled and lin.ks == 1 and (not rtw or lin.rtw == rtw)
    xa = decoder_ops.tile_rows(x) if x_tiled else x
    out = lin(xa, x_tiled=x_tiled, rows=rows)
    torch.cuda.synchronize()
    gate, up = _linear_ref(x, wg), _linear_ref(x, wu)
    ref = gate / (1 + torch.exp(-gate)) * up
    got = decoder_ops.untile_rows(out, rows)
    _check_linear(got, ref)
    assert torch.equal(lin.plain(), torch.cat([wg, wu], 0))


@pytest.mark.parametrize("ks,rows,dim", [(4, 64, 4096), (1, 64, 4096), (3, 5, 4096), (5, 64, 4096), (9, 2, 1000)])
def test_rmsnorm_residual_from_partials(gpu, ks, rows, dim):
    """res_part (a projection's fp32 split partials) gives h = bf16(x + sum of the slices, in slice order)
    and the norm of it; more than four slices take the kernel's extra load rounds, dim 1000 has lanes past
    the row's end."""
    g = torch.Generator().manual_seed(5 + ks)
    x = torch.randn(rows, dim, generator=g).to(gpu, torch.bfloat16)
    part = torch.randn(ks, rows, dim, generator=g).to(gpu)
    w = (1 + 0.1 * torch.randn(dim, generator=g)).to(gpu, torch.bfloat16)
    h = x.clone()
    y = decoder_ops.rmsnorm(h, w, 1e-5, res_part=part, h_out=h)
    torch.cuda.synchronize()
    s = part[0].clone()
    for k in range(1, ks):
        s += part[k]
    h_ref = (x.float() + s).to(torch.bfloat16)
    assert torch.equal(h, h_ref)
    hf = h_ref.float()
    y_ref = (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-5) * w.float())
    assert (y.float() - y_ref).abs().max() <= 2e-2 * y_ref.abs().max()


@pytest.mark.parametrize("layout,gs,r_k,r_v,k_rope", [("tiled", 1, 64, 96, False), ("rows", 1, 32, 128, False),
                                                      ("tiled", 4, 256, 192, False), ("tiled", 1, 128, 64, True),
                                                      ("tiled", 1, 80, 48, False)])
def test_qkv_post_equals_rope_and_appends(gpu, layout, gs, r_k, r_v, k_rope):
    """The fused QKV epilogue: q rotated at each row's position, every group's K and V slices appended at
    that position (rotated K for the stock path), from fp32 split partials; against rope of the summed
    projection and the strided appends of its bf16 rounding."""
    g = torch.Generator().manual_seed(r_k + r_v + gs)
    B, nh, nkv, hd, S, ks = 6, 8, 4, 128, 256, 3
    G = nkv // gs
    ncols = (nh + 2 * nkv) * hd
    part = torch.randn(ks, B, ncols, generator=g).to(gpu)
    pos = torch.tensor([0, 5, 31, 32, 200, 255], dtype=torch.int32, device=gpu)
    cos, sin = fused.cos_sin_tables(hd, S, 500000.0, None)
    cos, sin = cos.to(gpu).contiguous(), sin.to(gpu).contiguous()
    k_w = hd if k_rope else r_k
    mk = (lambda w, role: LatentCache.zeros(B, G, S, w, gpu, role)) if layout == "tiled" else \
        (lambda w, role: torch.zeros(B, G, S, w, dtype=torch.bfloat16, device=gpu))
    keys, values, keys2, values2 = mk(k_w, "k"), mk(r_v, "v"), mk(k_w, "k"), mk(r_v, "v")
    q = decoder_ops.qkv_post(part, pos, cos, sin, nh, keys, nh * hd, gs * hd, k_w, values, (nh + nkv) * hd, gs * hd, r_v,
                             k_rope=k_rope)
    s = part[0] + part[1] + part[2]
    xqkv = s.to(torch.bfloat16)
    if k_rope:
        krot = fused.apply_rope_meta(s[:, nh * hd:(nh + nkv) * hd].view(B, nkv, hd), cos[pos.long()][:, None],
                                     sin[pos.long()][:, None]).to(torch.bfloat16)
        decoder_ops.append_from(keys2, krot.reshape(B, nkv * hd), hd, hd, pos)
    else:
        decoder_ops.append_from(keys2, xqkv[:, nh * hd:], gs * hd, k_w, pos)
    decoder_ops.append_from(values2, xqkv[:, (nh + nkv) * hd:], gs * hd, r_v, pos)
    torch.cuda.synchronize()
    q_ref = fused.apply_rope_meta(s[:, :nh * hd].view(B, nh, hd), cos[pos.long()][:, None], sin[pos.long()][:, None])
    assert (q.float() - q_ref).abs().max() <= 1e-2 * q_ref.abs().max()
    kt = (lambda c: c.to_rows()) if layout == "tiled" else (lambda c: c)
    if k_rope:
        assert (kt(keys).float() - kt(keys2).float()).abs().max() <= 1e-2 * krot.float().abs().max()
    else:
        assert torch.equal(kt(keys), kt(keys2))
    assert torch.equal(kt(values), kt(values2))


@pytest.mark.parametrize("layout,gs,r_k,r_v,k_rope,rows,x_tiled,rtw",
                         [("tiled", 1, 64, 96, False, 6, True, 0), ("rows", 1, 32, 128, False, 6, False, 0),
                          ("tiled", 4, 256, 192, False, 6, True, 3), ("tiled", 1, 128, 64, True, 6, False, 0),
                          ("tiled", 1, 80, 48, False, 64, True, 0), ("tiled", 1, 112, 64, False, 33, True, 5)])
def test_linear_qkv_equals_projection_and_qkv_post(gpu, layout, gs, r_k, r_v, k_rope, rows, x_tiled, rtw):
    """The QKV projection with its epilogue in one launch: q and both caches bit for bit as the one-slice
    projection's fp32 output through qkv_post (same products, same order, same rotation and rounding)."""
    g = torch.Generator().manual_seed(r_k + r_v + gs + rows)
    nh, nkv, hd, S, dim = 8, 4, 128, 256, 1024
    G = nkv // gs
    k_w = hd if k_rope else r_k
    k0, v0 = nh * hd, nh * hd + G * k_w
    n = v0 + G * r_v
    x = torch.randn(rows, dim, generator=g).to(gpu, torch.bfloat16)
    w = (torch.randn(n, dim, generator=g) * 0.03).to(gpu, torch.bfloat16)
    pos = torch.randint(0, S, (rows,), generator=g).to(gpu, torch.int32)
    pos[0] = 0
    pos[-1] = S - 1
    cos, sin = fused.cos_sin_tables(hd, S, 500000.0, None)
    cos, sin = cos.to(gpu).contiguous(), sin.to(gpu).contiguous()
    mk = (lambda wd, role: LatentCache.zeros(rows, G, S, wd, gpu, role)) if layout == "tiled" else \
        (lambda wd, role: torch.zeros(rows, G, S, wd, dtype=torch.bfloat16, device=gpu))
    keys, values, keys2, values2 = mk(k_w, "k"), mk(r_v, "v"), mk(k_w, "k"), mk(r_v, "v")
    rtw = rtw or decoder_ops.linear_plan(rows, n, dim, 1)[0]
    wt = decoder_ops.tile_weight(w, rtw)
    xa = decoder_ops.tile_rows(x) if x_tiled else x
    q = decoder_ops.linear_qkv(xa, wt, rtw, pos, cos, sin, nh, keys, k0, k_w, k_w, values, v0, r_v, r_v,
                               k_rope=k_rope, x_tiled=x_tiled, rows=rows)
    part = decoder_ops.linear_tiled(xa, wt, rtw, 1, x_tiled=x_tiled, rows=rows, mode="partials")
    q2 = decoder_ops.qkv_post(part, pos, cos, sin, nh, keys2, k0, k_w, k_w, values2, v0, r_v, r_v, k_rope=k_rope)
    torch.cuda.synchronize()
    kt = (lambda c: c.to_rows()) if layout == "tiled" else (lambda c: c)
    assert torch.equal(q, q2)
    assert torch.equal(kt(keys), kt(keys2)) and torch.equal(kt(values), kt(values2))
    q_ref = fused.apply_rope_meta(_linear_ref(x, w)[:, :k0].view(rows, nh, hd), cos[pos.long()][:, None],
                                  sin[pos.long()][:, None])
    _check_linear(q, q_ref)


@pytest.mark.parametrize("layout", ["tiled", "rows"])
def test_linear_qkv_positions_outside_the_cache(gpu, layout):
    """Rows whose position lies outside the cache (negative, or at or past its length) get q rotated at the
    position (clamped into the rotation table) and append nothing, as qkv_post does; the other rows
    append as usual."""
    g = torch.Generator().manual_seed(77)
    nh, hd, S, dim, G, r = 4, 128, 64, 256, 2, 32
    k0, v0 = nh * hd, nh * hd + G * r
    n = v0 + G * r
    x = torch.randn(4, dim, generator=g).to(gpu, torch.bfloat16)
    w = (torch.randn(n, dim, generator=g) * 0.05).to(gpu, torch.bfloat16)
    pos = torch.tensor([-1, S, 3, S + 5], dtype=torch.int32, device=gpu)
    cos, sin = fused.cos_sin_tables(hd, S, 500000.0, None)
    cos, sin = cos.to(gpu).contiguous(), sin.to(gpu).contiguous()
    mk = (lambda wd, role: LatentCache.zeros(4, G, S, wd, gpu, role)) if layout == "tiled" else \
        (lambda wd, role: torch.zeros(4, G, S, wd, dtype=torch.bfloat16, device=gpu))
    keys, values, keys2, values2 = mk(r, "k"), mk(r, "v"), mk(r, "k"), mk(r, "v")
    rtw = decoder_ops.linear_plan(4, n, dim, 1)[0]
    wt = decoder_ops.tile_weight(w, rtw)
    q = decoder_ops.linear_qkv(x, wt, rtw, pos, cos, sin, nh, keys, k0, r, r, values, v0, r, r)
    part = decoder_ops.linear_tiled(x, wt, rtw, 1, mode="partials")
    q2 = decoder_ops.qkv_post(part, pos, cos, sin, nh, keys2, k0, r, r, values2, v0, r, r)
    torch.cuda.synchronize()
    kt = (lambda c: c.to_rows()) if layout == "tiled" else (lambda c: c)
    assert torch.equal(q, q2)
    assert torch.equal(kt(keys), kt(keys2)) and torch.equal(kt(values), kt(values2))
    rows = kt(keys).float().abs().sum(dim=(1, 3))                     # [B, S]: nonzero where appended
    assert rows[2, 3] > 0 and rows.count_nonzero() == 1
    clamp = pos.long().clamp(0, cos.shape[0] - 1)                     # the table's rows, not the cache's
    q_ref = fused.apply_rope_meta(_linear_ref(x, w)[:, :k0].view(4, nh, hd), cos[clamp][:, None], sin[clamp][:, None])
    _check_linear(q, q_ref)


def test_linear_qkv_rejects_overlapping_ranges(gpu):
    x = torch.zeros(4, 256, dtype=torch.bfloat16, device=gpu)
    wt = torch.zeros(128 + 2 * 64, 256, dtype=torch.bfloat16, device=gpu)
    pos = torch.zeros(4, dtype=torch.int32, device=gpu)
    cos, sin = fused.cos_sin_tables(128, 64, 500000.0, None)
    cos, sin = cos.to(gpu).contiguous(), sin.to(gpu).contiguous()
    keys = torch.zeros(4, 1, 64, 64, dtype=torch.bfloat16, device=gpu)
    values = torch.zeros(4, 1, 64, 64, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="must not overlap"):
        decoder_ops.linear_qkv(x, wt, 1, pos, cos, sin, 1, keys, 128, 64, 64, values, 160, 64, 64)
    with pytest.raises(RuntimeError, match="must not overlap"):
        decoder_ops.linear_qkv(x, wt, 1, pos, cos, sin, 1, keys, 64, 64, 64, values, 192, 64, 64)


@pytest.mark.parametrize("rows,n,k,x_tiled,with_tiled", [(64, 4096, 2048, True, True), (64, 4096, 4096, False, True),
                                                         (23, 4096, 1280, True, True), (5, 400, 1344, False, False)])
def test_linear_residual_equals_partials_plus_h(gpu, rows, n, k, x_tiled, with_tiled):
    """h += x w^T in the projection's epilogue: bit for bit bf16(h + the one-slice fp32 product), the tiled
    copy equal to tile_rows of the new h, rows past the live count of the tiled copy untouched."""
    g = torch.Generator().manual_seed(n + k + rows)
    x = torch.randn(rows, k, generator=g).to(gpu, torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.02).to(gpu, torch.bfloat16)
    h = torch.randn(rows, n, generator=g).to(gpu, torch.bfloat16)
    rtw = decoder_ops.linear_plan(rows, n, k, 1)[0]
    wt = decoder_ops.tile_weight(w, rtw)
    xa = decoder_ops.tile_rows(x) if x_tiled else x
    part = decoder_ops.linear_tiled(xa, wt, rtw, 1, x_tiled=x_tiled, rows=rows, mode="partials")
    h_ref = (h.float() + part[0]).to(torch.bfloat16)
    ht = torch.full((64, n), float("nan"), dtype=torch.bfloat16, device=gpu) if with_tiled else None
    hw = torch.zeros(rows, n + 8, dtype=torch.bfloat16, device=gpu)
    hv = hw[:, 4:4 + n]
    hv.copy_(h)
    decoder_ops.linear_residual(xa, wt, rtw, hv, ht, x_tiled=x_tiled, rows=rows)
    torch.cuda.synchronize()
    assert torch.equal(hv, h_ref)
    assert (hw[:, :4] == 0).all() and (hw[:, 4 + n:] == 0).all()
    _check_linear(part[0], _linear_ref(x, w))
    if with_tiled:
        assert torch.equal(decoder_ops.untile_rows(ht, rows), h_ref)
        pad = decoder_ops.untile_weight(ht, 4)[rows:]
        assert torch.isnan(pad.float()).all()


@pytest.mark.parametrize("rows,x_tiled,rtw", [(64, True, 0), (64, False, 0), (13, True, 0), (64, True, 7), (21, True, 5),
                                              (64, True, 2)])
def test_linear_swiglu_rmsnorm(gpu, rows, x_tiled, rtw):
    """The gate / up launch over RMS-normalised rows (norm weight folded into the gate / up columns) against
    fp32 torch: silu(g) * u of rmsnorm(x) w^T; and against palu_rmsnorm followed by the SwiGLU projection
    within their two bf16 roundings. Rows of the tiled input past the live count hold NaN and are ignored.
    rtw 7 (the decoder's gate / up split) and 5 leave an odd tile per wave and a short last group."""
    g = torch.Generator().manual_seed(rows + 7 * x_tiled + 100 * rtw)
    k, f, eps = 2048, 1536, 1e-5
    x = (torch.randn(rows, k, generator=g) * 3).to(gpu, torch.bfloat16)
    nw = (1 + 0.2 * torch.randn(k, generator=g)).to(gpu, torch.bfloat16)
    wg = (torch.randn(f, k, generator=g) * 0.05).to(gpu, torch.bfloat16)
    wu = (torch.randn(f, k, generator=g) * 0.05).to(gpu, torch.bfloat16)
    lin = decoder_ops.DecodeLinear(None, 64, gate_up=(wg, wu), in_scale=nw, rtw=rtw, ks=1 if rtw else 0)
    assert lin.tiled and lin.in_scale_folded and (not rtw or lin.rtw == rtw)
    if x_tiled:
        pad = torch.full((64, k), float("nan"), dtype=torch.bfloat16, device=gpu)
        pad[:rows] = x
        xa = decoder_ops.tile_weight(pad, 4)
    else:
        xa = x
    out = lin.swiglu_rmsnorm(xa, eps, x_tiled=x_tiled, rows=rows)
    plain = decoder_ops.DecodeLinear(None, 64, gate_up=(wg, wu))
    y = decoder_ops.rmsnorm(x, nw, eps)
    two = plain(y)
    torch.cuda.synchronize()
    got = decoder_ops.untile_rows(out, rows).float()
    xf = x.float()
    xn = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * nw.float()
    gate, up = xn @ wg.float().T, xn @ wu.float().T
    ref = gate / (1 + torch.exp(-gate)) * up
    scale = ref.abs().max().item()
    # the folded weight and the output each round once to bf16
    assert (got - ref).abs().max().item() <= scale * 2 ** -6
    assert F.cosine_similarity(got.flatten(), ref.flatten(), dim=0).item() >= 0.9999
    two = decoder_ops.untile_rows(two, rows).float()
    assert (got - two).abs().max().item() <= scale * 2 ** -5


@pytest.mark.parametrize("B,S,r_k,r_v,hpg", [(32, 512, 64, 64, 1), (3, 1024, 96, 32, 1), (16, 256, 128, 256, 4)])
def test_sdpa_decode_tiled_rows_output(gpu, B, S, r_k, r_v, hpg):
    """palu_sdpa_decode with tiled_rows writes tile_rows of its row-major output, bit for bit (fixed
    block order): items in one chunk (B = 32: 256 items), items merged from chunks (B = 3), and the
    grouped-latent path (u_v, 128-wide output)."""
    g = torch.Generator().manual_seed(B * 100 + r_k)
    nh, nkv, hd = 32, 8, 128
    ng = nkv // hpg
    q = torch.randn(1, B, nh, hd, generator=g).to(gpu, torch.bfloat16)
    k = torch.randn(B, ng, S, r_k, generator=g).to(gpu, torch.bfloat16)
    v = torch.randn(B, ng, S, r_v, generator=g).to(gpu, torch.bfloat16)
    u_k = (torch.randn(nkv, r_k, hd, generator=g) / r_k ** 0.5).to(torch.bfloat16)
    u_v = (torch.randn(1, nkv, r_v, hd, generator=g) / r_v ** 0.5).to(gpu, torch.bfloat16) if hpg > 1 else None
    pos = torch.randint(0, S, (B,), generator=g).to(gpu, torch.int32)
    cos, sin = fused.cos_sin_tables(hd, S, 500000.0, None)
    w_rot = fused.w_rot_from_u_k(u_k).to(gpu, torch.bfloat16)[None]
    cs = fused.cs_table(cos, sin, S)[None, None].to(gpu)
    kc, vc = LatentCache.from_rows(k, "k"), LatentCache.from_rows(v, "v")
    width = hd if hpg > 1 else r_v
    a = fused.palu_sdpa_decode(q, kc, w_rot, cs, vc, width, pos, u_v=u_v, deterministic=True)
    t = fused.palu_sdpa_decode(q, kc, w_rot, cs, vc, width, pos, u_v=u_v, deterministic=True, tiled_rows=True)
    torch.cuda.synchronize()
    assert t.shape == (64, nh * width)
    assert torch.equal(decoder_ops.untile_rows(t, B), a[0].reshape(B, nh * width))
