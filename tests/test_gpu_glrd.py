"""GPU parity of the grouped-latent path (G-LRD): heads_per_group KV heads share one K latent and one V
latent, every KV head rebuilds K with its own u_k slice and V with its own u_v slice in-kernel
(palu_sdpa_decode with u_v; reference interface docs/superpowers/specs/2026-09-12-palu-tt-stage2b-
design.md:120-142). Oracle: reference_decode with u_v (fp32), on the same bf16-rounded inputs; bar
max-abs 2e-2 and cosine 0.9999. Group ranks cover the configuration's set {128, 192, 256, 384, 512}; the
caches are tiled (LatentCache), compact per group (GroupedLatentCache) or the reference's row-major tensors.
"""
import pytest
import torch

from oracle import palu_oracle as ref
from palu_tt import decoder_ops, fused
from palu_tt.cache import GroupedLatentCache, LatentCache

pytestmark = pytest.mark.gpu

HD = 128
THETA = 500000.0
LLAMA3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}


def _bf(t):
    return t.to(torch.bfloat16).float()


def _case(B, S, r_k, r_v, hpg, seed, nh=32, nkv=8, pos=None):
    g = torch.Generator().manual_seed(seed)
    ng = nkv // hpg
    q = _bf(torch.randn(1, B, nh, HD, generator=g))
    k = _bf(torch.randn(B, ng, S, r_k, generator=g))
    v = _bf(torch.randn(B, ng, S, r_v, generator=g))
    u_k = _bf(torch.randn(nkv, r_k, HD, generator=g) / r_k ** 0.5)
    u_v = _bf(torch.randn(nkv, r_v, HD, generator=g) / r_v ** 0.5)
    if pos is None:
        pos = torch.randint(0, S, (B,), generator=g)
        pos[0] = S - 1
        if B > 2:
            pos[1], pos[2] = 0, 127
    return q, k, v, u_k, u_v, pos


def _run(dev, q, k, v, u_k, u_v, pos, S, out_dtype=torch.float32, cs_dtype=torch.float32, **kw):
    cos, sin = fused.cos_sin_tables(HD, S, THETA, LLAMA3)
    out = fused.palu_sdpa_decode(
        q.to(dev, torch.bfloat16), LatentCache.from_rows(k.to(dev, torch.bfloat16), "k"),
        fused.w_rot_from_u_k(u_k).to(dev, torch.bfloat16)[None], fused.cs_table(cos, sin, S)[None, None].to(dev, cs_dtype),
        LatentCache.from_rows(v.to(dev, torch.bfloat16), "v"), HD, pos.to(dev, torch.int32),
        u_v=u_v.to(dev, torch.bfloat16)[None], scale=HD ** -0.5, out_dtype=out_dtype, **kw)
    torch.cuda.synchronize()
    return out.float().cpu()


def _run_rows(dev, q, k, v, u_k, u_v, pos, S, out_dtype=torch.float32, rope=LLAMA3, **kw):
    """The reference's own call: plain row-major [B, n_groups, S, r] latent tensors
    (tests/test_palu_sdpa_device.py:245-258), no cache object."""
    cos, sin = fused.cos_sin_tables(HD, S, THETA, rope)
    out = fused.palu_sdpa_decode(
        q.to(dev, torch.bfloat16), k.to(dev, torch.bfloat16).contiguous(),
        fused.w_rot_from_u_k(u_k).to(dev, torch.bfloat16)[None], fused.cs_table(cos, sin, S)[None, None].to(dev),
        v.to(dev, torch.bfloat16).contiguous(), HD, pos.to(dev, torch.int32), u_v=u_v.to(dev, torch.bfloat16)[None],
        scale=HD ** -0.5, out_dtype=out_dtype, **kw)
    torch.cuda.synchronize()
    return out.float().cpu()


def _oracle(q, k, v, u_k, u_v, pos, S):
    cos, sin = ref.cos_sin_tables(HD, S, THETA, LLAMA3)
    return ref.reference_decode(q, k, u_k, v, pos, cos, sin, HD ** -0.5, u_v=u_v)


def _check(out, exp, max_abs=2e-2, cos=0.9999):
    ma, cs = ref.max_abs(out, exp), ref.cosine(out, exp)
    assert torch.isfinite(out).all() and ma <= max_abs and cs >= cos, f"max_abs {ma:.3e}, cosine {cs:.6f}"


@pytest.mark.parametrize("r_k,r_v", [(128, 128), (192, 256), (256, 192), (384, 512), (512, 512), (512, 128)])
def test_glrd_matches_oracle_group_ranks(gpu, r_k, r_v):
    """Two groups of four KV heads (heads_per_group 4), the configuration's group ranks."""
    args = _case(4, 1024, r_k, r_v, hpg=4, seed=r_k + r_v)
    _check(_run(gpu, *args, 1024), _oracle(*args, 1024))


@pytest.mark.parametrize("hpg,r_k,r_v", [(1, 64, 96), (2, 160, 32), (8, 96, 320)])
def test_glrd_other_group_sizes_and_ranks(gpu, hpg, r_k, r_v):
    """Per-head latents with in-kernel V (group size 1), group sizes 2 and 8, ranks that are not
    multiples of 64."""
    args = _case(3, 640, r_k, r_v, hpg=hpg, seed=hpg * 1000 + r_k)
    _check(_run(gpu, *args, 640), _oracle(*args, 640))


@pytest.mark.parametrize("B,S", [(1, 4096), (2, 300), (5, 33)])
def test_glrd_splits_and_ragged_lengths(gpu, B, S):
    """Batch 1 splits every sequence across workgroups (merged by the out kernel); lengths that are
    not a multiple of the 32-position block and caches shorter than one block group."""
    S_pad = (S + 31) // 32 * 32
    args = list(_case(B, S_pad, 256, 256, hpg=4, seed=B * 7 + S))
    args[5] = torch.minimum(args[5], torch.tensor(S - 1))
    _check(_run(gpu, *args, S_pad), _oracle(*args, S_pad))


def test_glrd_bf16_output_and_table(gpu):
    args = _case(4, 512, 192, 192, hpg=4, seed=99)
    exp = _oracle(*args, 512)
    _check(_run(gpu, *args, 512, out_dtype=torch.bfloat16), exp)
    _check(_run(gpu, *args, 512, cs_dtype=torch.bfloat16), exp, max_abs=5e-2, cos=0.999)


def test_glrd_row_major_bf16_output_and_table(gpu):
    """The reference's row-major call with a bf16 output and a bf16 [cos | sin] table."""
    args = _case(4, 512, 192, 192, hpg=4, seed=98)
    exp = _oracle(*args, 512)
    _check(_run_rows(gpu, *args, 512, out_dtype=torch.bfloat16), exp)
    cos, sin = fused.cos_sin_tables(HD, 512, THETA, LLAMA3)
    q, k, v, u_k, u_v, pos = args
    out = fused.palu_sdpa_decode(
        q.to(gpu, torch.bfloat16), k.to(gpu, torch.bfloat16), fused.w_rot_from_u_k(u_k).to(gpu, torch.bfloat16)[None],
        fused.cs_table(cos, sin, 512)[None, None].to(gpu, torch.bfloat16), v.to(gpu, torch.bfloat16), HD,
        pos.to(gpu, torch.int32), u_v=u_v.to(gpu, torch.bfloat16)[None], scale=HD ** -0.5, out_dtype=torch.float32)
    torch.cuda.synchronize()
    _check(out.cpu(), exp, max_abs=5e-2, cos=0.999)


def test_glrd_reference_head_shape(gpu):
    """The reference op tests' per-chip shape: 16 Q / 4 KV heads, one group of 4."""
    args = _case(8, 1024, 256, 384, hpg=4, seed=5, nh=16, nkv=4)
    _check(_run(gpu, *args, 1024), _oracle(*args, 1024))


@pytest.mark.parametrize("ranks", [None, (512, 384), (512, 512)])
def test_glrd_configuration_shape(gpu, ranks):
    """Batch 16, ctx 16384, 2 groups of 4 heads, group ranks drawn from {128, 192, 256, 384, 512}, and
    the two layers the benchmark times (the drawn widest pair (512, 384), and (512, 512)); the oracle
    checks 3 of the 16 rows (the kernel computes all of them in one call)."""
    g = torch.Generator().manual_seed(4)
    choices = [128, 192, 256, 384, 512]
    r_k = choices[int(torch.randint(0, 5, (1,), generator=g))]
    r_v = choices[int(torch.randint(0, 5, (1,), generator=g))]
    if ranks is not None:
        r_k, r_v = ranks
    B, S = 16, 16384
    q, k, v, u_k, u_v, pos = _case(B, S, r_k, r_v, hpg=4, seed=44, pos=torch.full((16,), S - 1))
    pos[3], pos[9] = 5000, 12345
    out = _run(gpu, q, k, v, u_k, u_v, pos, S)
    rows = [0, 3, 9]
    exp = _oracle(q[:, rows], k[rows], v[rows], u_k, u_v, pos[rows], S)
    _check(out[:, rows], exp)


@pytest.mark.parametrize("S,pos", [(49152, [49151, 40000, 16383]), (65536, [65535, 32768, 16384])])
def test_glrd_widest_ranks_at_long_context(gpu, S, pos):
    """r_k = r_v = 512 (u_k^T of 128 KB in LDS) at contexts past 40k and at the 65536 maximum: every
    pair base angle comes from the three small angle tables (no table grows with the context). Rows end
    at the last position, mid-cache and on 16384-position boundaries (where the top table's row
    changes); all three rows are checked."""
    B = len(pos)
    q, k, v, u_k, u_v, p = _case(B, S, 512, 512, hpg=4, seed=S, pos=torch.tensor(pos))
    _check(_run(gpu, q, k, v, u_k, u_v, p, S), _oracle(q, k, v, u_k, u_v, p, S))


@pytest.mark.parametrize("ranks_k,ranks_v,B,S", [([128, 512], [192, 384], 16, 16384), ([96, 32], [64, 160], 3, 1000),
                                                  ([256, 256], [512, 128], 2, 4096)])
def test_glrd_per_group_ranks_never_read_the_padding(gpu, ranks_k, ranks_v, B, S):
    """Groups of unequal ranks in caches padded to the widest group: told each group's own ranks, the op
    reads and multiplies only those columns. The padding columns of the latents and the padding rows of
    u_k / u_v hold NaN on the GPU (zeros for the oracle), so a single read of them would show. The first
    case is the configuration's drawn layer (B=16, ctx 16384, K ranks (128, 512), V ranks (192, 384))."""
    S32 = (S + 31) // 32 * 32
    r_k, r_v = max(ranks_k), max(ranks_v)
    q, k, v, u_k, u_v, pos = _case(B, S32, r_k, r_v, hpg=4, seed=sum(ranks_k) + S)
    pos.clamp_(max=S - 1)
    for g, (rk, rv) in enumerate(zip(ranks_k, ranks_v)):
        k[:, g, :, rk:] = 0
        v[:, g, :, rv:] = 0
        u_k[4 * g:4 * g + 4, rk:] = 0
        u_v[4 * g:4 * g + 4, rv:] = 0
    rows = [0, B - 1] if B > 2 else list(range(B))
    exp = _oracle(q[:, rows], k[rows], v[rows], u_k, u_v, pos[rows], S32)
    kn, vn, ukn, uvn = k.clone(), v.clone(), u_k.clone(), u_v.clone()
    for g, (rk, rv) in enumerate(zip(ranks_k, ranks_v)):
        kn[:, g, :, rk:] = float("nan")
        vn[:, g, :, rv:] = float("nan")
        ukn[4 * g:4 * g + 4, rk:] = float("nan")
        uvn[4 * g:4 * g + 4, rv:] = float("nan")
    out = _run(gpu, q, kn, vn, ukn, uvn, pos, S32, group_ranks=(ranks_k, ranks_v))
    _check(out[:, rows], exp)


@pytest.mark.parametrize("ranks_k,ranks_v,B,S", [([128, 512], [192, 384], 4, 4096), ([96, 32], [64, 160], 3, 1000),
                                                  ([256, 256], [512, 128], 2, 2048)])
def test_glrd_compact_group_caches(gpu, ranks_k, ranks_v, B, S):
    """Every group stored at its own ranks (GroupedLatentCache, PALU_LAYOUT_TILED_GROUPED): the decode
    equals, bit for bit, the one over caches padded to the widest group and told the group ranks, and
    matches the oracle; appends land in each group's own stream (checked through to_rows); the storage
    is the groups' own bytes."""
    S32 = (S + 31) // 32 * 32
    r_k, r_v = max(ranks_k), max(ranks_v)
    q, k, v, u_k, u_v, pos = _case(B, S32, r_k, r_v, hpg=4, seed=sum(ranks_v) + S)
    pos.clamp_(max=S - 1)
    for g, (rk, rv) in enumerate(zip(ranks_k, ranks_v)):
        k[:, g, :, rk:] = 0
        v[:, g, :, rv:] = 0
        u_k[4 * g:4 * g + 4, rk:] = 0
        u_v[4 * g:4 * g + 4, rv:] = 0
    gk = GroupedLatentCache.from_rows(k.to(gpu, torch.bfloat16), ranks_k, "k")
    gv = GroupedLatentCache.from_rows(v.to(gpu, torch.bfloat16), ranks_v, "v")
    assert gk.nbytes() + gv.nbytes() == B * S32 * (sum(ranks_k) + sum(ranks_v)) * 2
    # append one new row per batch row at its position, from a strided source wider than every rank
    new_k = _bf(torch.randn(B, 2, r_k + 32))
    new_v = _bf(torch.randn(B, 2, r_v + 32))
    dpos = pos.to(gpu, torch.int32)
    decoder_ops.append_from(gk, new_k.to(gpu, torch.bfloat16).reshape(B, -1), r_k + 32, r_k + 32, dpos)
    decoder_ops.append_from(gv, new_v.to(gpu, torch.bfloat16).reshape(B, -1), r_v + 32, r_v + 32, dpos)
    for b in range(B):
        for g, (rk, rv) in enumerate(zip(ranks_k, ranks_v)):
            k[b, g, pos[b], :rk] = new_k[b, g, :rk]
            v[b, g, pos[b], :rv] = new_v[b, g, :rv]
    torch.cuda.synchronize()
    assert torch.equal(gk.to_rows().float().cpu(), k) and torch.equal(gv.to_rows().float().cpu(), v)
    cos, sin = fused.cos_sin_tables(HD, S32, THETA, LLAMA3)
    compact = fused.palu_sdpa_decode(
        q.to(gpu, torch.bfloat16), gk, fused.w_rot_from_u_k(u_k).to(gpu, torch.bfloat16)[None],
        fused.cs_table(cos, sin, S32)[None, None].to(gpu), gv, HD, dpos, u_v=u_v.to(gpu, torch.bfloat16)[None],
        scale=HD ** -0.5, out_dtype=torch.float32)
    torch.cuda.synchronize()
    padded = _run(gpu, q, k, v, u_k, u_v, pos, S32, group_ranks=(ranks_k, ranks_v))
    assert torch.equal(compact.cpu(), padded)
    rows = [0, B - 1]
    _check(padded[:, rows], _oracle(q[:, rows], k[rows], v[rows], u_k, u_v, pos[rows], S32))


def test_glrd_deterministic_repeat(gpu):
    args = _case(2, 2048, 256, 256, hpg=4, seed=8)
    a = _run(gpu, *args, 2048)
    b = _run(gpu, *args, 2048)
    assert torch.equal(a, b)


def test_pinned_heads_per_core_that_does_not_fit_the_grid_is_rejected(gpu):
    """A pinned heads_per_core is checked against the program config's core grid
    (reference tests/test_palu_sdpa_device.py:490-503): batch 4 of one group of 4 KV heads on a 2 x 2
    grid, 2 heads per core, wants 8 cores and is rejected before any launch; 4 heads per core (the whole
    group on one core, 4 items) fits and decodes to the oracle."""
    args = _case(4, 256, 128, 128, hpg=4, seed=21, nh=16, nkv=4)
    cfg = fused.SDPAProgramConfig(compute_with_storage_grid_size=(2, 2), k_chunk_size=128)
    with pytest.raises(RuntimeError, match="only 4 available"):
        _run(gpu, *args, 256, heads_per_core=2, program_config=cfg)
    _check(_run(gpu, *args, 256, heads_per_core=4, program_config=cfg), _oracle(*args, 256))


# ---- the reference's own G-LRD call: row-major [B, n_groups, S, r] latents ---------------------------

def _reference_group_case(batch, S, r_k, r_v, gs, seed, nh=16, nkv=4):
    """Inputs of the reference's _inputs_group (tests/test_palu_sdpa_device.py:219-232): its per-chip
    16 Q / 4 KV heads, latents and queries N(0, 1), factors N(0, 1/r), positions uniform with row 0 at
    S - 1 and, from batch 4 on, rows 1-3 at 0, 127 and 128."""
    g = torch.Generator().manual_seed(seed)
    ng = nkv // gs
    q = _bf(torch.randn(1, batch, nh, HD, generator=g))
    k = _bf(torch.randn(batch, ng, S, r_k, generator=g))
    u_k = _bf(torch.randn(nkv, r_k, HD, generator=g) / r_k ** 0.5)
    v = _bf(torch.randn(batch, ng, S, r_v, generator=g))
    u_v = _bf(torch.randn(nkv, r_v, HD, generator=g) / r_v ** 0.5)
    pos = torch.randint(0, S, (batch,), generator=g)
    pos[0] = S - 1
    if batch >= 4:
        pos[1], pos[2], pos[3] = 0, 127, 128
    return q, k, v, u_k, u_v, pos


def _oracle_plain(q, k, v, u_k, u_v, pos, S):
    cos, sin = ref.cos_sin_tables(HD, S, THETA, None)
    return ref.reference_decode(q, k, u_k, v, pos, cos, sin, HD ** -0.5, u_v=u_v)


@pytest.mark.parametrize("batch,S,r_k,r_v,gs", [
    (1, 1024, 128, 256, 4), (32, 1024, 128, 256, 4),       # test_grouped_latents_with_in_kernel_v (:278-281)
    (1, 1024, 256, 512, 4), (32, 1024, 256, 512, 4),
    (1, 1024, 384, 512, 4), (32, 1024, 384, 512, 4),
    (8, 8192, 64, 512, 4),                                 # test_grouped_latents_long_context_batch8 (:298-299)
    (32, 1024, 64, 64, 1),                                 # test_in_kernel_v_with_per_head_latents (:302-304)
    (32, 1024, 512, 512, 4),                               # test_grouped_latents_full_rank_group (:316-318)
])
def test_glrd_reference_row_major_call(gpu, batch, S, r_k, r_v, gs):
    """The reference's G-LRD op cases as it calls them: row-major latents, u_v, head_dim_v 128, its
    per-chip head shape and input distributions, plain RoPE tables; every row against the oracle at
    the op's bar (max-abs 2e-2, cosine 0.9999)."""
    args = _reference_group_case(batch, S, r_k, r_v, gs, seed=batch * 1000 + r_k + r_v + gs)
    out = _run_rows(gpu, *args, S, rope=None)
    assert out.shape == (1, batch, 16, HD)
    _check(out, _oracle_plain(*args, S))


@pytest.mark.parametrize("r_k,r_v,B,S", [(128, 192, 4, 2048), (512, 384, 2, 4096), (96, 160, 3, 640)])
def test_glrd_row_major_equals_tiled(gpu, r_k, r_v, B, S):
    """Row-major and tiled caches holding the same latents give the same output bit for bit: the same
    scores arithmetic, and the row-major V pieces are moved into the tiled operand order exactly
    (identity products), so the PV sums are the same."""
    args = _case(B, S, r_k, r_v, hpg=4, seed=r_k * 3 + r_v + S)
    assert torch.equal(_run_rows(gpu, *args, S), _run(gpu, *args, S))


@pytest.mark.parametrize("ranks_k,ranks_v,B,S", [([128, 512], [192, 384], 4, 4096), ([96, 32], [64, 160], 3, 1000)])
def test_glrd_row_major_group_ranks_and_ragged_cache(gpu, ranks_k, ranks_v, B, S):
    """Row-major caches padded to the widest group, told each group's ranks, with NaN in every padding
    column and in every cache row past each row's position (never attended): only a group's own
    columns and the attended rows are read into a result. S = 1000 is not a multiple of the 32-position
    block, so the last block's rows past the cache end are clamped to its last row and masked."""
    r_k, r_v = max(ranks_k), max(ranks_v)
    q, k, v, u_k, u_v, pos = _case(B, S, r_k, r_v, hpg=4, seed=sum(ranks_k) * 7 + S)
    pos[0] = S - 1
    for g, (rk, rv) in enumerate(zip(ranks_k, ranks_v)):
        k[:, g, :, rk:] = 0
        v[:, g, :, rv:] = 0
        u_k[4 * g:4 * g + 4, rk:] = 0
        u_v[4 * g:4 * g + 4, rv:] = 0
    exp = _oracle(q, k, v, u_k, u_v, pos, S)
    kn, vn = k.clone(), v.clone()
    for g, (rk, rv) in enumerate(zip(ranks_k, ranks_v)):
        kn[:, g, :, rk:] = float("nan")
        vn[:, g, :, rv:] = float("nan")
    for b in range(B):
        kn[b, :, int(pos[b]) + 1:] = float("nan")
        vn[b, :, int(pos[b]) + 1:] = float("nan")
    _check(_run_rows(gpu, q, kn, vn, u_k, u_v, pos, S, group_ranks=(ranks_k, ranks_v)), exp)


def test_glrd_compact_caches_at_the_benchmark_shape(gpu):
    """The layer the benchmark times (B=16, ctx 16384, 2 groups of 4 KV heads, K ranks (128, 512), V
    ranks (192, 384), each group stored at its own ranks in GroupedLatentCaches) against the oracle
    on three rows, two of them ending mid-cache; the same call on the row-major padded caches (the
    reference's form) gives the same bits."""
    ranks_k, ranks_v = [128, 512], [192, 384]
    B, S = 16, 16384
    q, k, v, u_k, u_v, pos = _case(B, S, 512, 384, hpg=4, seed=16384, pos=torch.full((16,), S - 1))
    pos[7], pos[15] = 9000, 16000
    for g, (rk, rv) in enumerate(zip(ranks_k, ranks_v)):
        k[:, g, :, rk:] = 0
        v[:, g, :, rv:] = 0
        u_k[4 * g:4 * g + 4, rk:] = 0
        u_v[4 * g:4 * g + 4, rv:] = 0
    kd, vd = k.to(gpu, torch.bfloat16), v.to(gpu, torch.bfloat16)
    gk = GroupedLatentCache.from_rows(kd, ranks_k, "k")
    gv = GroupedLatentCache.from_rows(vd, ranks_v, "v")
    cos, sin = fused.cos_sin_tables(HD, S, THETA, LLAMA3)
    compact = fused.palu_sdpa_decode(
        q.to(gpu, torch.bfloat16), gk, fused.w_rot_from_u_k(u_k).to(gpu, torch.bfloat16)[None],
        fused.cs_table(cos, sin, S)[None, None].to(gpu), gv, HD, pos.to(gpu, torch.int32),
        u_v=u_v.to(gpu, torch.bfloat16)[None], scale=HD ** -0.5, out_dtype=torch.float32)
    torch.cuda.synchronize()
    compact = compact.cpu()
    del gk, gv
    rows_out = _run_rows(gpu, q, kd, vd, u_k, u_v, pos, S, group_ranks=(ranks_k, ranks_v))
    assert torch.equal(compact, rows_out)
    rows = [0, 7, 15]
    _check(compact[:, rows], _oracle(q[:, rows], k[rows], v[rows], u_k, u_v, pos[rows], S))


def test_glrd_32_groups_of_unequal_ranks(gpu):
    """Per-head latents with u_v at 32 KV heads (32 latent groups, the most the grouped-latent kernels
    take), each group at its own drawn K and V ranks in compact caches: the PV pass deals its splits over
    32 groups of different widths and the group tables are full. Against the oracle, and bit for bit
    against row-major caches padded to the widest group."""
    B, S, nkv = 3, 768, 32
    g = torch.Generator().manual_seed(3232)
    ranks_k = [int(x) * 32 for x in torch.randint(1, 5, (nkv,), generator=g)]
    ranks_v = [int(x) * 32 for x in torch.randint(1, 5, (nkv,), generator=g)]
    ranks_k[0], ranks_v[1] = 128, 128
    q, k, v, u_k, u_v, pos = _case(B, S, max(ranks_k), max(ranks_v), hpg=1, seed=3233, nh=32, nkv=nkv)
    for gi, (rk, rv) in enumerate(zip(ranks_k, ranks_v)):
        k[:, gi, :, rk:] = 0
        v[:, gi, :, rv:] = 0
        u_k[gi, rk:] = 0
        u_v[gi, rv:] = 0
    gk = GroupedLatentCache.from_rows(k.to(gpu, torch.bfloat16), ranks_k, "k")
    gv = GroupedLatentCache.from_rows(v.to(gpu, torch.bfloat16), ranks_v, "v")
    cos, sin = fused.cos_sin_tables(HD, S, THETA, LLAMA3)
    compact = fused.palu_sdpa_decode(
        q.to(gpu, torch.bfloat16), gk, fused.w_rot_from_u_k(u_k).to(gpu, torch.bfloat16)[None],
        fused.cs_table(cos, sin, S)[None, None].to(gpu), gv, HD, pos.to(gpu, torch.int32),
        u_v=u_v.to(gpu, torch.bfloat16)[None], scale=HD ** -0.5, out_dtype=torch.float32)
    torch.cuda.synchronize()
    compact = compact.float().cpu()
    rows = _run_rows(gpu, q, k, v, u_k, u_v, pos, S, group_ranks=(ranks_k, ranks_v))
    assert torch.equal(compact, rows)
    _check(compact, _oracle(q, k, v, u_k, u_v, pos, S))
