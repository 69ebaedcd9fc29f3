"""Host-side logic of palu_tt against the oracle, and the C-ABI library on a machine without a GPU.

Nothing here launches a kernel: the C-ABI checks load the library, compare its exports with the
declarations in include/palu_mi355x.h, and drive argument validation, which the library finishes before
it touches the HIP runtime.
"""
import ctypes
import json
import re
from pathlib import Path

import pytest
import torch
from safetensors.torch import save_file

from oracle import palu_oracle as ref
from palu_tt import _build, _native, compress, convert, fused

REPO = Path(__file__).resolve().parents[1]
HD = 128
THETA = 500000.0
LLAMA3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}


# ------------------------------------------------------------------------------------------------
# Tables (palu_tt/fused.py:36-79 of the reference)

def test_table_builders_equal_the_oracle():
    for scaling in (LLAMA3, None):
        assert torch.equal(fused.rope_frequencies(HD, THETA, scaling), ref.inv_freq(HD, THETA, scaling))
        c1, s1 = fused.cos_sin_tables(HD, 2048, THETA, scaling)
        c0, s0 = ref.cos_sin_tables(HD, 2048, THETA, scaling)
        assert torch.equal(c1, c0) and torch.equal(s1, s0)
    c, s = ref.cos_sin_tables(HD, 1024, THETA, LLAMA3)
    assert torch.equal(fused.cs_table(c, s, 1000), ref.cs_table(c, s, 1000))
    assert torch.equal(fused.rot_step_table(c, s, 256), ref.rot_step_table(c, s, 256))
    assert torch.equal(fused.rope_transformation_matrix(HD), ref.rope_transformation_matrix(HD))
    assert torch.equal(fused.trans_mat_tile()[0, 0], ref.rope_transformation_matrix(HD)[:32, :32])
    u = torch.randn(2, 64, HD)
    torch.testing.assert_close(fused.w_rot_from_u_k(u), ref.w_rot_from_u_k(u))
    for S in (1, 96, 256, 1000, 1024, 8192, 8224, 65536):
        assert fused.chunk_size(S) == ref.chunk_size(S)
    x = torch.randn(3, 5, HD)
    torch.testing.assert_close(fused.apply_rope_meta(x, c[:5], s[:5]), ref.meta_rotate(x, c[:5], s[:5]))


# ------------------------------------------------------------------------------------------------
# Weight layout (palu_tt/convert.py of the reference)

def test_reverse_permute_equals_the_oracle():
    W = torch.randn(4 * 16, 7)
    assert torch.equal(convert.reverse_permute(W, 4, 64, 7), ref.reverse_permute(W, 4, 64, 7))


def _layer(seed, hidden=256, nh=4, nkv=2, hd=HD):
    g = torch.Generator().manual_seed(seed)
    return {"q": torch.randn(nh * hd, hidden, generator=g) * 0.05, "k": torch.randn(nkv * hd, hidden, generator=g) * 0.05,
            "v": torch.randn(nkv * hd, hidden, generator=g) * 0.05, "o": torch.randn(hidden, nh * hd, generator=g) * 0.05}


@pytest.mark.parametrize("r_k,r_v", [(32, 64), (64, 32), (HD, 64), (32, HD)])
def test_converted_decode_tensors_reproduce_the_layer_oracle(r_k, r_v):
    """M-LRD: latents from wk/wv_lat_pad, the op model on (u_k, v latent), wo_fused on the r_v-wide output
    padded to hd == the HF-convention layer oracle's decode step. Covers the full-rank collapses (r == hd)."""
    hidden, nh, nkv, T = 256, 4, 2, 9
    W = _layer(r_k + r_v)
    Uk, VTk = ref.svd_per_head(W["k"], nkv, r_k)
    Uv, VTv = ref.svd_per_head(W["v"], nkv, r_v)
    lr = convert.LowRank(VTk, Uk, VTv, Uv)
    t = convert.palu_layer_tensors(W, lr, nh, nkv, HD)
    x = torch.randn(1, T, hidden)
    layer = ref.PaluRefAttention(nh, nkv, HD, THETA, LLAMA3, W["q"], W["o"], ref.Factors(VTk, Uk, VTv, Uv))
    layer.forward(x[:, :-1], 0)
    exp = layer.forward(x[:, -1:], T - 1)[0, 0]

    kl = (x[0] @ t["wk_lat_pad"].T).view(T, nkv, HD)          # per KV head, the first r_k columns
    vl = (x[0] @ t["wv_lat_pad"].T).view(T, nkv, HD)
    if r_k == HD:                                               # full K rows (Meta order), u_k = I
        k_lat, u_k = kl.permute(1, 0, 2)[None], torch.eye(HD).expand(nkv, HD, HD)
    else:
        k_lat, u_k = kl[..., :r_k].permute(1, 0, 2)[None], t["u_k"]
        assert torch.equal(t["w_rot"][..., :HD], u_k)
    v_lat = vl[..., :r_v].permute(1, 0, 2)[None] if r_v != HD else vl.permute(1, 0, 2)[None]
    q = (x[0, -1] @ W["q"].T).view(nh, HD)
    cq, sq = ref.hf_cos_sin(torch.tensor([T - 1]), HD, THETA, LLAMA3)
    q = q * cq + ref.rotate_half(q) * sq
    q_meta = torch.stack([ref.reverse_permute(q[h][:, None], 1, HD, 1)[:, 0] for h in range(nh)])
    cos, sin = ref.cos_sin_tables(HD, T, THETA, LLAMA3)
    o = ref.reference_decode(q_meta[None, None], k_lat, u_k, v_lat, torch.tensor([T - 1]), cos, sin, HD ** -0.5)
    o_pad = torch.zeros(nh, HD)
    o_pad[:, :o.shape[-1]] = o[0, 0]
    torch.testing.assert_close(o_pad.reshape(-1) @ t["wo_fused"].T, exp, atol=2e-5, rtol=1e-4)


def _write_palu_dir(path: Path, layers, hidden, hd, groups_k, groups_v, seed=0):
    """A Palu factor directory in the on-disk format load_palu_dir reads (reference compress.py:37-46)."""
    g = torch.Generator().manual_seed(seed)
    ranks, tensors = {}, {}
    for i in range(layers):
        for proj, groups in (("k_proj", groups_k), ("v_proj", groups_v)):
            key = f"model.layers.{i}.self_attn.{proj}"
            gs = len(groups[0][1])
            ranks[key] = [r for r, _ in groups]
            tensors[f"{key}.VT.weight"] = torch.randn(sum(r for r, _ in groups), hidden, generator=g)
            for gi, (r, _) in enumerate(groups):
                tensors[f"{key}.U.{gi}.weight"] = torch.randn(gs * hd, r, generator=g)
    path.mkdir(parents=True, exist_ok=True)
    (path / "config.json").write_text(json.dumps({"head_wise_ranks": ranks}))
    save_file(tensors, str(path / "palu_lowrank.safetensors"))
    return ranks, tensors


def test_load_palu_dir_mlrd_and_glrd(tmp_path):
    hidden, hd, nkv = 64, 16, 4
    mlrd = [(24, [0]), (40, [1]), (8, [2]), (32, [3])]            # group size 1, ragged ranks
    glrd = [(48, [0, 1]), (20, [2, 3])]                           # 2 groups of 2 heads
    ranks, tensors = _write_palu_dir(tmp_path / "m", 1, hidden, hd, mlrd, glrd)
    with pytest.raises(ValueError, match="group size"):
        convert.load_palu_dir(tmp_path / "m", 1, nkv, hd)
    ranks, tensors = _write_palu_dir(tmp_path / "g", 2, hidden, hd, glrd, glrd)
    lr = convert.load_palu_dir(tmp_path / "g", 2, nkv, hd, rank_multiple=32)
    assert set(lr) == {0, 1} and lr[0].group_size == 2 and lr[0].r_k == 64     # 48 padded up to 64
    assert lr[1].group_ranks_k == [48, 20] and lr[1].group_ranks_v == [48, 20]
    key = "model.layers.1.self_attn.k_proj"
    VT_all = tensors[f"{key}.VT.weight"]
    for h in range(nkv):
        gi = h // 2
        r = ranks[key][gi]
        off = sum(ranks[key][:gi])
        assert torch.equal(lr[1].k_VT[h, :r], VT_all[off:off + r])
        assert torch.count_nonzero(lr[1].k_VT[h, r:]) == 0 and torch.count_nonzero(lr[1].k_U[h, :, r:]) == 0
        U_g = tensors[f"{key}.U.{gi}.weight"]
        assert torch.equal(lr[1].k_U[h, :, :r], U_g[(h % 2) * hd:(h % 2 + 1) * hd])
    u = convert.load_palu_dir(tmp_path / "g", 2, nkv, hd, latent_scale="unit")
    for h in range(nkv):
        torch.testing.assert_close(u[0].k_U[h] @ u[0].k_VT[h], lr[0].k_U[h] @ lr[0].k_VT[h], atol=1e-4, rtol=1e-4)
    assert torch.count_nonzero(u[0].k_U[2:, :, 20:]) == 0          # rank padding stays zero
    # with balanced SVD factors (U = U_r sqrt(S), VT = sqrt(S) V_r^T) unit scaling leaves VT orthonormal,
    # i.e. unit-variance latents for white inputs (reference tests/test_convert.py:453-484)
    W = torch.randn(nkv * hd, hidden)
    U, VT = ref.svd_per_head(W, nkv, 12)
    s = convert.unit_scale_lowrank(convert.LowRank(VT, U, VT.clone(), U.clone()))
    for h in range(nkv):
        torch.testing.assert_close(s.k_VT[h] @ s.k_VT[h].T, torch.eye(12), atol=1e-4, rtol=0)
        torch.testing.assert_close(s.k_U[h] @ s.k_VT[h], U[h] @ VT[h], atol=1e-4, rtol=1e-4)
    assert convert.palu_dir_cache_id(tmp_path / "g").startswith("g-")
    assert convert.palu_cache_id_for(tmp_path / "g", "unit").endswith("-unit")


def test_palu_dir_round_trip_reproduces_the_weights_at_full_rank(tmp_path):
    """compress.factor_layers -> convert.save_palu_dir -> convert.load_palu_dir: at full rank (r = group
    rows) every head's U @ VT is its own rows of W, for per-head (M-LRD) and grouped (G-LRD) factors; at
    ragged ranks the loaded head equals the truncated group SVD's slice, zero-padded."""
    hidden, hd, nkv = 96, 16, 4
    g = torch.Generator().manual_seed(3)
    W = {i: {"k": torch.randn(nkv * hd, hidden, generator=g), "v": torch.randn(nkv * hd, hidden, generator=g)}
         for i in range(2)}
    for gs in (1, 2):
        ng = nkv // gs
        full = [[gs * hd] * ng] * 2
        d = convert.save_palu_dir(tmp_path / f"full{gs}", compress.factor_layers(W, nkv, full, full))
        lr = convert.load_palu_dir(d, 2, nkv, hd, rank_multiple=16)
        for i in range(2):
            assert lr[i].group_size == gs and lr[i].r_k == gs * hd
            for h in range(nkv):
                torch.testing.assert_close(lr[i].k_U[h] @ lr[i].k_VT[h], W[i]["k"][h * hd:(h + 1) * hd],
                                           atol=2e-4, rtol=1e-4)
                torch.testing.assert_close(lr[i].v_U[h] @ lr[i].v_VT[h], W[i]["v"][h * hd:(h + 1) * hd],
                                           atol=2e-4, rtol=1e-4)
    ragged_k, ragged_v = [[10, 7], [16, 3]], [[5, 12], [9, 9]]
    fac = compress.factor_layers(W, nkv, ragged_k, ragged_v)
    d = convert.save_palu_dir(tmp_path / "ragged", fac, meta={"note": "ragged"})
    assert json.loads((d / "config.json").read_text())["head_wise_ranks"]["model.layers.1.self_attn.k_proj"] == [16, 3]
    lr = convert.load_palu_dir(d, 2, nkv, hd, rank_multiple=8)
    assert lr[0].r_k == 16 and lr[1].r_v == 16 and lr[1].r_k == 16
    for h in range(nkv):
        gi, hh = divmod(h, 2)
        U_g, VT_g = fac[1]["k_proj"][gi]
        r = VT_g.shape[0]
        assert torch.equal(lr[1].k_VT[h, :r], VT_g) and torch.count_nonzero(lr[1].k_VT[h, r:]) == 0
        assert torch.equal(lr[1].k_U[h, :, :r], U_g[hh * hd:(hh + 1) * hd]) and torch.count_nonzero(lr[1].k_U[h, :, r:]) == 0
    # the balanced split matches the oracle's per-head SVD (group size 1)
    U, VT = compress.svd_per_head(W[0]["k"], nkv, 5)
    Ur, VTr = ref.svd_per_head(W[0]["k"], nkv, 5)
    torch.testing.assert_close(U @ VT, Ur @ VTr, atol=1e-4, rtol=1e-4)


def test_group_ranks_off_the_kernel_grid_round_up_to_32():
    """A dump's group ranks are any positive integers (config.json head_wise_ranks); the layer hands the
    fused op and its compact caches each rank rounded up to 32, capped at the padded width, with the
    widest group at exactly that width (load_palu_dir pads r_k / r_v from the widest raw rank)."""
    from palu_tt.attention import kernel_group_ranks
    assert kernel_group_ranks([100, 140], [176, 96], 160, 192) == ([128, 160], [192, 96])     # rank_multiple 32
    assert kernel_group_ranks([100, 140], [176, 96], 192, 192) == ([128, 192], [192, 96])     # rank_multiple 64
    assert kernel_group_ranks([8, 4], [8, 4], 32, 32) == ([32, 32], [32, 32])
    assert kernel_group_ranks([128, 512], [192, 384], 512, 384) == ([128, 512], [192, 384])   # already on the grid
    assert kernel_group_ranks([33, 500, 31], [1, 1, 64], 512, 64) == ([64, 512, 32], [32, 32, 64])


def test_palu_dir_cache_id_tracks_content(tmp_path):
    """The id is dirname-<8 hex>, stable across reads and file touches, and changes when one byte of
    config.json changes or the tensors are regenerated with the same shapes."""
    import os
    import re
    groups = [(32, [0]), (32, [1]), (32, [2]), (32, [3])]
    d = tmp_path / "my dump 0.5"
    _write_palu_dir(d, 1, 64, 32, groups, groups, seed=1)
    cid = convert.palu_dir_cache_id(d)
    assert re.fullmatch(r"my_dump_0\.5-[0-9a-f]{8}", cid), cid
    shard = d / "palu_lowrank.safetensors"
    os.utime(shard, ns=(1, 1))
    assert convert.palu_dir_cache_id(d) == cid
    cj = d / "config.json"
    cj.write_text(cj.read_text() + " ")
    cid2 = convert.palu_dir_cache_id(d)
    assert cid2 != cid and cid2.startswith("my_dump_0.5-")
    _write_palu_dir(d, 1, 64, 32, groups, groups, seed=2)
    assert convert.palu_dir_cache_id(d) not in (cid, cid2)
    assert convert.palu_cache_id_for(d, "balanced") == convert.palu_dir_cache_id(d)


def test_add_palu_to_state_dict_from_hf_and_palu_dirs(tmp_path):
    """The converter over an HF checkpoint directory: identity factors without a dump (cache id
    "identity", stock collapse: wo_fused == wo), and a dump's factors laid out per layer as
    palu_layer_tensors lays them (reference convert.py:291-312 is the interface)."""
    hidden, nh, nkv, L = 256, 8, 4, 2
    g = torch.Generator().manual_seed(5)
    hf_dir = tmp_path / "hf"
    hf_dir.mkdir()
    Ws = {i: _layer(10 + i, hidden, nh, nkv) for i in range(L)}
    save_file({f"model.layers.{i}.self_attn.{p}_proj.weight": w[p].contiguous() for i, w in Ws.items()
               for p in "qkvo"} | {"model.embed_tokens.weight": torch.randn(16, hidden, generator=g)},
              str(hf_dir / "model.safetensors"))
    w1 = convert.hf_attn_weights(hf_dir, 1)
    assert set(w1) == {"q", "k", "v", "o"} and torch.equal(w1["k"], Ws[1]["k"])
    with pytest.raises(KeyError):
        convert.hf_attn_weights(hf_dir, 5)
    sd = {}
    cfg = convert.add_palu_to_state_dict(sd, hf_dir, None, L, nh, nkv, HD)
    assert cfg.cache_id == "identity" and cfg.rank_k == [HD, HD] and cfg.group_size == 1
    assert torch.equal(sd["layers.0.attention.palu.wo_fused"], Ws[0]["o"].float())
    ranks = [[64] * nkv, [32] * nkv]
    pd = convert.save_palu_dir(tmp_path / "dump", compress.factor_layers({i: Ws[i] for i in range(L)}, nkv, ranks, ranks))
    sd = {}
    cfg = convert.add_palu_to_state_dict(sd, hf_dir, pd, L, nh, nkv, HD)
    assert cfg.rank_k == [64, 32] and cfg.rank_v == [64, 32] and cfg.cache_id.startswith("dump-")
    lrs = convert.load_palu_dir(pd, L, nkv, HD)
    for i in range(L):
        exp = convert.palu_layer_tensors(Ws[i], lrs[i], nh, nkv, HD)
        for k, t in exp.items():
            assert torch.equal(sd[f"layers.{i}.attention.palu.{k}"], t), (i, k)


def test_glrd_layer_tensors_share_the_group_latent_and_keep_wo():
    hidden, nh, nkv, gs, r = 256, 8, 4, 2, 64
    W = _layer(5, hidden, nh, nkv)
    Uk, VTk = ref.svd_per_head(W["k"], nkv, r)
    Uv, VTv = ref.svd_per_head(W["v"], nkv, r)
    for h in range(1, nkv, 2):                 # heads of one group carry the group's VT
        VTk[h], VTv[h] = VTk[h - 1], VTv[h - 1]
    t = convert.palu_layer_tensors(W, convert.LowRank(VTk, Uk, VTv, Uv, group_size=gs), nh, nkv, HD)
    assert torch.equal(t["wo_fused"], W["o"])
    assert torch.equal(t["wk_lat_pad"][:r], VTk[0]) and torch.count_nonzero(t["wk_lat_pad"][HD:2 * HD]) == 0
    assert torch.equal(t["wk_lat_pad"][2 * HD:2 * HD + r], VTk[2])
    assert t["u_v"].shape == (nkv, r, HD) and torch.equal(t["u_v"][1], Uv[1].T)


# ------------------------------------------------------------------------------------------------
# The C-ABI library without a GPU

def _declared_functions():
    text = (REPO / "include" / "palu_mi355x.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(palu_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    if not _build.library_path().exists():
        _build.build_native()
    return _native.load()


def test_library_exports_every_declared_function(lib):
    names = _declared_functions()
    assert names == sorted(_native.EXPORTED), f"header declares {names}, binding has {sorted(_native.EXPORTED)}"
    raw = ctypes.CDLL(str(_build.library_path()))
    for n in names:
        assert getattr(raw, n) is not None
    assert lib.palu_abi_version() == _native.ABI_VERSION
    hdr = (REPO / "include" / "palu_mi355x.h").read_text()
    assert f"#define PALU_ABI_VERSION {_native.ABI_VERSION}" in hdr


def test_workspace_query(lib):
    # the headline shape (256 items on 256 CUs) needs no split; a long single row splits
    assert lib.palu_decode_workspace_bytes(32, 8, 8192, 64) == 0
    ws = lib.palu_decode_workspace_bytes(1, 8, 65536, 64)
    assert ws > 0 and ws % 4 == 0
    assert lib.palu_decode_workspace_bytes(0, 8, 8192, 64) == 0


def test_grouped_latent_workspace_query(lib):
    # scores ([B, n_q, S] fp32) plus the PV partials
    B, nq, nkv, G, S, rv = 16, 32, 8, 2, 16384, 512
    ws = lib.palu_glrd_workspace_bytes(B, nq, nkv, G, S, rv)
    assert ws >= B * nq * S * 4 and ws < B * nq * S * 4 + B * nq * 129 * (rv + 4) * 4 + 512
    assert lib.palu_glrd_workspace_bytes(B, nq, nkv, 3, S, rv) == 0          # groups must divide the KV heads
    assert lib.palu_glrd_workspace_bytes(0, nq, nkv, G, S, rv) == 0


_FAKE = ctypes.c_void_p(1 << 20)          # aligned, never dereferenced: validation fails before any use


def _sdpa(lib, **kw):
    a = dict(q=_FAKE, k=_FAKE, w=_FAKE, cs=_FAKE, v=_FAKE, head_dim_v=64, cur=_FAKE, out=_FAKE, rot_step=None,
             trans_mat=None, u_v=None, group_ranks=None, scale=0.088, heads_per_core=0, rot_mode=2, table_mcast=1, k_chunk=0,
             batch=2, n_q=8, n_kv=2, n_groups=2, seq_len=256, r_k=64, r_v=64, w_rot_width=256, cs_rows=256,
             cs_cols=256, cs_dtype=0, out_dtype=1, layout=0, det=0, ws=None, ws_bytes=0, stream=None)
    a.update(kw)
    rc = lib.palu_sdpa_decode(a["q"], a["k"], a["w"], a["cs"], a["v"], a["head_dim_v"], a["cur"], a["out"],
                              a["rot_step"], a["trans_mat"], a["u_v"], a["group_ranks"], a["scale"], a["heads_per_core"],
                              a["rot_mode"],
                              a["table_mcast"], a["k_chunk"], a["batch"], a["n_q"], a["n_kv"], a["n_groups"],
                              a["seq_len"], a["r_k"], a["r_v"], a["w_rot_width"], a["cs_rows"], a["cs_cols"],
                              a["cs_dtype"], a["out_dtype"], a["layout"], a["det"], a["ws"], a["ws_bytes"], a["stream"])
    return rc, lib.palu_last_error().decode()


@pytest.mark.parametrize("kw,code,needle", [
    (dict(r_k=48), _native.PALU_EINVAL, "r_k"),
    (dict(r_k=40, layout=1), _native.PALU_EINVAL, "r_k must be a multiple of 16"),
    (dict(cs_cols=128), _native.PALU_EINVAL, "cs_tab"),
    (dict(cs_rows=100), _native.PALU_EINVAL, "cs_tab"),
    (dict(w_rot_width=128), _native.PALU_EINVAL, "w_rot"),
    (dict(rot_step=_FAKE), _native.PALU_EINVAL, "optional together"),
    (dict(k_chunk=256), _native.PALU_EINVAL, "Phase 1"),
    (dict(rot_mode=5), _native.PALU_EINVAL, "rot_mode must be"),
    (dict(n_groups=3, n_kv=4), _native.PALU_EINVAL, "heads_per_group"),
    (dict(u_v=_FAKE, head_dim_v=64), _native.PALU_EINVAL, "head_dim_v"),
    (dict(u_v=_FAKE, head_dim_v=128), _native.PALU_EINVAL, "palu_glrd_workspace_bytes"),   # rows accepted
    (dict(layout=3), _native.PALU_EINVAL, "needs u_v and group_ranks"),
    (dict(head_dim_v=128), _native.PALU_EINVAL, "head_dim_v"),
    (dict(heads_per_core=4), _native.PALU_EINVAL, "heads_per_core"),
    (dict(n_q=6, n_kv=4, n_groups=4), _native.PALU_EINVAL, "KV head count"),
    (dict(n_kv=4, n_groups=2), _native.PALU_EINVAL, "u_v"),                 # grouped V latent without u_v
    (dict(heads_per_core=2), _native.PALU_EINVAL, "grouped latents"),     # per-head latents cannot be shared
    (dict(heads_per_core=8, n_q=16, n_kv=4, n_groups=2), _native.PALU_EINVAL, "KV head count"),
    (dict(heads_per_core=4, n_q=16, n_kv=4, n_groups=2), _native.PALU_EINVAL, "heads_per_group"),
    (dict(layout=1, seq_len=100, cs_rows=100), _native.PALU_EINVAL, "multiple of 32"),
    (dict(seq_len=70000, cs_rows=70000), _native.PALU_EUNSUPPORTED, "65536"),
    (dict(q=ctypes.c_void_p((1 << 20) + 2)), _native.PALU_EINVAL, "aligned"),
    (dict(out=None), _native.PALU_EINVAL, "null"),
    (dict(group_ranks=(ctypes.c_int32 * 4)(32, 64, 64, 64)), _native.PALU_EUNSUPPORTED, "group_ranks"),
    (dict(group_ranks=(ctypes.c_int32 * 4)(48, 64, 64, 64)), _native.PALU_EINVAL, "multiple of 32"),
    (dict(group_ranks=(ctypes.c_int32 * 4)(64, 64, 96, 64)), _native.PALU_EINVAL, "V rank"),
])
def test_sdpa_decode_envelope_errors(lib, kw, code, needle):
    rc, msg = _sdpa(lib, **kw)
    assert rc == code and needle in msg, (rc, msg)


def test_flash_decode_and_append_envelope_errors(lib):
    rc = lib.palu_flash_decode(_FAKE, _FAKE, _FAKE, _FAKE, _FAKE, 0.1, 2, 6, 4, 256, 128, 1, 0, 0, None, 0, None)
    assert rc == _native.PALU_EINVAL and "KV head count" in lib.palu_last_error().decode()
    rc = lib.palu_flash_decode(_FAKE, _FAKE, _FAKE, _FAKE, _FAKE, 0.1, 2, 8, 2, 100, 128, 1, 1, 0, None, 0, None)
    assert rc == _native.PALU_EINVAL and "multiple of 32" in lib.palu_last_error().decode()
    rc = lib.palu_latent_append(_FAKE, _FAKE, _FAKE, 2, 2, 256, 12, 0, None)
    assert rc == _native.PALU_EINVAL and "multiple of 8" in lib.palu_last_error().decode()
    rc = lib.palu_latent_append(_FAKE, _FAKE, _FAKE, 2, 2, 256, 40, 1, None)
    assert rc == _native.PALU_EINVAL and "multiple of 16" in lib.palu_last_error().decode()
    widths = (ctypes.c_int32 * 2)(64, 40)
    rc = lib.palu_latent_append_grouped(_FAKE, _FAKE, 256, 128, _FAKE, 2, 2, 256, widths, 1, None)
    assert rc == _native.PALU_EINVAL and "group 1 width 40" in lib.palu_last_error().decode()
    widths = (ctypes.c_int32 * 2)(64, 32)
    rc = lib.palu_latent_append_grouped(_FAKE, _FAKE, 256, 128, _FAKE, 2, 2, 256, widths, 0, None)
    assert rc == _native.PALU_EINVAL and "order must be" in lib.palu_last_error().decode()
    rc = lib.palu_latent_append_grouped(_FAKE, _FAKE, 256, 128, _FAKE, 2, 33, 256, widths, 1, None)
    assert rc == _native.PALU_EINVAL and "1..32 groups" in lib.palu_last_error().decode()


def test_fused_projection_plans_and_envelope_errors(lib):
    """The one-slice plan the fused epilogues use, and their argument checks (host-side, before any launch)."""
    rtw, ks = ctypes.c_int(0), ctypes.c_int(0)
    assert lib.palu_linear_plan_ks(64, 5120, 4096, 1, ctypes.byref(rtw), ctypes.byref(ks)) == _native.PALU_OK
    assert ks.value == 1 and 1 <= rtw.value <= 8
    assert lib.palu_linear_plan_ks(64, 4096, 14336, 16, ctypes.byref(rtw), ctypes.byref(ks)) == _native.PALU_OK
    assert ks.value > 1
    assert lib.palu_linear_plan_ks(64, 4096, 14336, 0, ctypes.byref(rtw), ctypes.byref(ks)) == _native.PALU_EINVAL
    F = _FAKE
    rc = lib.palu_linear_swiglu_rmsnorm(F, 0, 1, 64, F, 4096 + 32, 4096, 7, 1e-5, F, None)
    assert rc == _native.PALU_EINVAL and "multiple of 64" in lib.palu_last_error().decode()
    rc = lib.palu_linear_residual(F, 0, 1, 64, F, 4096, 2048, 1, F, 4090, F, None)
    assert rc == _native.PALU_EINVAL and "ldh" in lib.palu_last_error().decode()
    rc = lib.palu_linear_residual(F, 0, 1, 65, F, 4096, 2048, 1, F, 4096, F, None)
    assert rc == _native.PALU_EINVAL and "1..64" in lib.palu_last_error().decode()
    # q heads 0..1023, K slices from 1024 (2 groups of 64), V slices overlapping the second K slice
    qkv = lambda v_off, k_gs=64: lib.palu_linear_qkv(F, 0, 1, 8, F, 1024 + 256, 1024, 1, F, F, F, 256, 8, F, F, 1, 1024,
                                                     k_gs, 64, 0, F, 2, v_off, 64, 64, 2, 256, None)
    assert qkv(1120) == _native.PALU_EINVAL and "must not overlap" in lib.palu_last_error().decode()
    assert qkv(1152, k_gs=32) == _native.PALU_EINVAL and "must not overlap" in lib.palu_last_error().decode()
    rc = lib.palu_linear_qkv(F, 0, 1, 8, F, 1280, 1024, 1, F, F, F, 256, 8, F, F, 2, 1024, 64, 64, 0, F, 2, 1152, 64,
                             64, 2, 256, None)
    assert rc == _native.PALU_EINVAL and "K caches are" in lib.palu_last_error().decode()


def test_paged_envelope_errors(lib):
    pt = _FAKE

    def sdpa_paged(page_table=pt, num_pages=16, page_size=64, max_pages=4, **kw):
        a = dict(head_dim_v=64, r_k=64, r_v=64, n_groups=2, n_kv=2, cs_rows=256, layout=0)
        a.update(kw)
        rc = lib.palu_sdpa_decode_paged(_FAKE, _FAKE, _FAKE, _FAKE, _FAKE, a["head_dim_v"], _FAKE, page_table, _FAKE,
                                        None, None, None, 0.088, 0, 2, 1, 0, 2, 8, a["n_kv"], a["n_groups"], num_pages,
                                        page_size, max_pages, a["r_k"], a["r_v"], 256, a["cs_rows"], 256, 0, 1,
                                        a["layout"], 0, None, 0, None)
        return rc, lib.palu_last_error().decode()

    assert sdpa_paged(page_table=None) == (_native.PALU_EINVAL, "palu_sdpa_decode_paged: page_table is null")
    rc, msg = sdpa_paged(page_size=48)
    assert rc == _native.PALU_EINVAL and "power of two" in msg
    rc, msg = sdpa_paged(page_size=16)
    assert rc == _native.PALU_EINVAL and "page_size" in msg
    rc, msg = sdpa_paged(num_pages=0)
    assert rc == _native.PALU_EINVAL and "num_pages" in msg
    rc, msg = sdpa_paged(max_pages=2048, cs_rows=131072)
    assert rc == _native.PALU_EUNSUPPORTED and "65536" in msg
    rc, msg = sdpa_paged(cs_rows=200)              # logical length 4 * 64 = 256 > 200 table rows
    assert rc == _native.PALU_EINVAL and "cs_tab" in msg
    rc, msg = sdpa_paged(r_k=48)
    assert rc == _native.PALU_EINVAL and "r_k" in msg
    rc = lib.palu_flash_decode_paged(_FAKE, _FAKE, _FAKE, _FAKE, None, _FAKE, 0.1, 2, 8, 2, 16, 64, 4, 128, 1, 0, 0,
                                     None, 0, None)
    assert rc == _native.PALU_EINVAL and "page_table" in lib.palu_last_error().decode()
    rc = lib.palu_latent_append_paged(_FAKE, _FAKE, _FAKE, _FAKE, 2, 2, 16, 96, 4, 64, 0, None)
    assert rc == _native.PALU_EINVAL and "power of two" in lib.palu_last_error().decode()
    rc = lib.palu_latent_append_paged(_FAKE, _FAKE, _FAKE, _FAKE, 2, 2, 16, 64, 4, 40, 1, None)
    assert rc == _native.PALU_EINVAL and "multiple of 16" in lib.palu_last_error().decode()
    rc, msg = sdpa_paged(r_k=40, layout=1)         # tiled caches: K widths in 16s
    assert rc == _native.PALU_EINVAL and "r_k must be a multiple of 16" in msg


def test_glrd_envelope_errors(lib):
    """Grouped latents with u_v: head_dim_v must be 128, r_k / r_v up to 512, caches contiguous (not
    paged). Row-major caches (the reference's call) pass the envelope and stop at the missing
    workspace, before any launch."""
    rc, msg = _sdpa(lib, u_v=_FAKE, head_dim_v=128, n_kv=4, n_groups=1, n_q=16, layout=0)
    assert rc == _native.PALU_EINVAL and "palu_glrd_workspace_bytes" in msg
    rc, msg = _sdpa(lib, u_v=_FAKE, head_dim_v=64, n_kv=4, n_groups=1, n_q=16, layout=1)
    assert rc == _native.PALU_EINVAL and "head_dim_v" in msg
    rc, msg = _sdpa(lib, u_v=_FAKE, head_dim_v=128, r_k=544, layout=1)
    assert rc == _native.PALU_EINVAL and "r_k" in msg
    # per-head latents with u_v: 32 groups are taken (they stop at the workspace), 64 are not
    rc, msg = _sdpa(lib, u_v=_FAKE, head_dim_v=128, n_q=64, n_kv=32, n_groups=32, layout=1)
    assert rc == _native.PALU_EINVAL and "palu_glrd_workspace_bytes" in msg
    rc, msg = _sdpa(lib, u_v=_FAKE, head_dim_v=128, n_q=64, n_kv=64, n_groups=64, layout=1)
    assert rc == _native.PALU_EUNSUPPORTED and "64 latent groups" in msg
    rc = lib.palu_sdpa_decode_paged(_FAKE, _FAKE, _FAKE, _FAKE, _FAKE, 128, _FAKE, _FAKE, _FAKE, None, None, _FAKE,
                                    0.088, 0, 2, 1, 0, 2, 16, 4, 1, 16, 64, 4, 256, 256, 256, 256, 256, 0, 1, 1, 0,
                                    None, 0, None)
    assert rc == _native.PALU_EUNSUPPORTED and "paged" in lib.palu_last_error().decode()


def test_bench_reads_the_committed_counter_summaries():
    """The bench line's roofline.traffic and mfma.busy_counter come from committed rocprofv3 summaries;
    both keys must be present and plausible (traffic at least the algorithmic latent bytes)."""
    import importlib.util
    root = Path(__file__).resolve().parent.parent
    spec = importlib.util.spec_from_file_location("bench_mod", root / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    traffic = bench.read_traffic(root / "profiles" / "palu_decode_b32_ctx8192_r64_traffic.txt")
    busy = bench.read_profile_value(root / "profiles" / "palu_decode_mfma_counters.md", "mfma_busy_headline")
    algorithmic = 32 * 8 * 8192 * (64 + 64) * 2
    assert traffic is not None and algorithmic <= traffic < 1.1 * algorithmic
    assert busy is not None and 0.0 < busy < 1.0
    assert bench.read_profile_value(root / "profiles" / "palu_decode_mfma_counters.md", "no_such_key") is None


def test_bench_refuses_more_than_one_gpu():
    import subprocess
    import sys
    root = Path(__file__).resolve().parent.parent
    res = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=300)
    assert res.returncode == 2
    assert "exactly one GPU" in json.loads(res.stdout.strip().splitlines()[-1])["error"]


def test_tile_weight_layout_and_inverse():
    """tile_weight puts w[16 rt + i][32 kt + 8 g + e] at lane 16 g + i, element e of tile (rt, kt) (the A
    operand of one 16x16x32 MFMA per 1 KB tile); row tiles form groups of rtw (the last one shorter when
    rtw does not divide them) stored [kt][rt in group]; untile_weight undoes it."""
    from palu_tt import decoder_ops
    n, k = 80, 96                                    # 5 row tiles, 3 k tiles
    w = torch.arange(n * k, dtype=torch.float32).reshape(n, k)
    n16, kt_n = n // 16, k // 32
    for rtw in (1, 2, 3, 5, 8):
        t = decoder_ops.tile_weight(w, rtw).reshape(-1)
        for rt in range(n16):
            grp, r = divmod(rt, rtw)
            cnt = min(rtw, n16 - grp * rtw)
            for kt in range(kt_n):
                for g, i, e in [(0, 0, 0), (3, 15, 7), (1, 4, 5), (2, 9, 2)]:
                    tile = grp * rtw * kt_n + kt * cnt + r
                    assert t[(tile * 64 + 16 * g + i) * 8 + e] == w[16 * rt + i, 32 * kt + 8 * g + e], (rtw, rt, kt)
        assert torch.equal(decoder_ops.untile_weight(decoder_ops.tile_weight(w, rtw), rtw), w)
    with pytest.raises(RuntimeError, match="n % 16"):
        decoder_ops.tile_weight(torch.zeros(40, 64), 1)
    with pytest.raises(RuntimeError, match="rtw"):
        decoder_ops.tile_weight(torch.zeros(32, 64), 9)
