"""The attention drop-in (palu_tt.attention.PaluAttention) against the HF-convention layer oracle.

A random Llama-shaped layer is compressed with per-head SVD (or per-group SVD for grouped latents),
converted with convert.palu_layer_tensors, and driven through prefill (two users) and several decode
steps; every output is compared with oracle.PaluRefAttention (fp32, same factors, same positions).
The layer runs in bf16 (weights, activations, caches), so the bar is on the whole layer output:
cosine >= 0.999 and max-abs within 2% of the output's largest magnitude. Covers the fused latent path
(r < head_dim), the naive path the reference runs when PaluRuntime.use_fused_k is off (K rebuilt and
rotated on the GPU, then the stock flash-decode; reference attention.py:657-710), the full-rank fast
paths (stock K / stock V), grouped latents with in-kernel V, and both cache layouts.
"""
import pytest
import torch

from oracle import palu_oracle as ref
from palu_tt import compress, convert
from palu_tt.attention import PaluAttention
from palu_tt.cache import GroupedLatentCache

pytestmark = pytest.mark.gpu

HD = 128
THETA = 500000.0
LLAMA3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}


class _Args:
    def __init__(self, dim, nh, nkv, max_seq, max_batch, palu):
        self.dim, self.n_heads, self.n_kv_heads, self.head_dim = dim, nh, nkv, HD
        self.max_seq_len, self.max_batch_size = max_seq, max_batch
        self.rope_theta, self.rope_scaling = THETA, LLAMA3
        self.palu = palu


def _group_svd(W, nkv, gs, rank, group_ranks=None):
    """Per-group truncated SVD with Palu's balanced split; every head of a group gets the group's VT
    and its hd-row slice of the group's U (reference compress.py:12-23, stage2b-design.md:80-86). With
    group_ranks, group g keeps its first group_ranks[g] components and is zero-padded to rank."""
    Wg = W.reshape(nkv // gs, gs * HD, -1)
    U, VT = ref.svd_per_head(Wg.reshape(-1, W.shape[1]), nkv // gs, rank)       # [G, gs*hd, r], [G, r, dim]
    for g, r in enumerate(group_ranks or []):
        U[g, :, r:] = 0
        VT[g, r:] = 0
    U_h = U.reshape(nkv // gs, gs, HD, rank).reshape(nkv, HD, rank)
    VT_h = VT.repeat_interleave(gs, dim=0)
    return U_h.contiguous(), VT_h.contiguous()


def _layer(dim, nh, nkv, r_k, r_v, gs, seed, use_fused_k=True, recon_len=None, group_ranks=None):
    g = torch.Generator().manual_seed(seed)
    W = {"q": torch.randn(nh * HD, dim, generator=g) * 0.02, "k": torch.randn(nkv * HD, dim, generator=g) * 0.02,
         "v": torch.randn(nkv * HD, dim, generator=g) * 0.02, "o": torch.randn(dim, nh * HD, generator=g) * 0.02}
    Uk, VTk = _group_svd(W["k"], nkv, gs, r_k, group_ranks and group_ranks[0])
    Uv, VTv = _group_svd(W["v"], nkv, gs, r_v, group_ranks and group_ranks[1])
    lr = convert.LowRank(VTk, Uk, VTv, Uv, group_size=gs)
    # the model state dict holds wq in Meta (interleaved-pair) order, as the reference's checkpoint loader
    # leaves it; the converter's K tensors are Meta-ordered too
    sd = {"layers.0.attention.wq.weight": convert.reverse_permute(W["q"], nh, nh * HD, dim),
          "layers.0.attention.wo.weight": W["o"]}
    for name, t in convert.palu_layer_tensors(W, lr, nh, nkv, HD).items():
        sd[f"layers.0.attention.palu.{name}"] = t
    palu = convert.PaluConfig(rank_k=[r_k], rank_v=[r_v], cache_id="test", group_size=gs,
                              runtime=convert.PaluRuntime(use_fused_k=use_fused_k, recon_len=recon_len, check=True),
                              group_ranks=[group_ranks] if group_ranks else None)
    oracle = ref.PaluRefAttention(nh, nkv, HD, THETA, LLAMA3, W["q"], W["o"], ref.Factors(VTk, Uk, VTv, Uv))
    return sd, palu, oracle


def _close(out, exp, what):
    out, exp = out.float().cpu(), exp.float()
    cs = ref.cosine(out, exp)
    rel = ref.max_abs(out, exp) / float(exp.abs().max())
    assert cs >= 0.999 and rel <= 0.02, f"{what}: cosine {cs:.6f}, max-abs / max {rel:.4f}"


@pytest.mark.parametrize("r_k,r_v,gs,layout,fused,recon_len", [
    (64, 64, 1, "tiled", True, None), (64, 64, 1, "rows", True, None), (32, 96, 1, "tiled", True, None),
    (HD, 64, 1, "tiled", True, None), (32, HD, 1, "tiled", True, None), (HD, HD, 1, "rows", True, None),
    (192, 256, 2, "tiled", True, None), (192, 256, 2, "rows", True, None),
    (64, 64, 1, "tiled", False, None), (32, 96, 1, "rows", False, 50), (192, 256, 2, "tiled", False, None),
    (32, HD, 1, "tiled", False, 64)])
def test_attention_prefill_then_decode_matches_layer_oracle(gpu, r_k, r_v, gs, layout, fused, recon_len):
    dim, nh, nkv, B, S0, steps = 1024, 8, 2, 2, 40, 6
    sd, palu, oracle = _layer(dim, nh, nkv, r_k, r_v, gs, seed=r_k + r_v + gs, use_fused_k=fused, recon_len=recon_len)
    _drive(gpu, sd, palu, oracle, dim, nh, nkv, B, S0, steps, layout, fused)


@pytest.mark.parametrize("fused", [True, False])
def test_attention_grouped_latents_of_unequal_ranks(gpu, fused):
    """G-LRD with 2 groups of 2 KV heads whose ranks differ (K 96 / 192, V 256 / 64), padded to the
    widest in the factors as load_palu_dir pads them; the layer keeps each group's latents at its own
    ranks (compact caches) and passes the groups' ranks to the fused op; the naive path rebuilds from
    the same compact caches."""
    dim, nh, nkv, B, S0, steps = 1024, 8, 4, 2, 40, 6
    gr = ([96, 192], [256, 64])
    sd, palu, oracle = _layer(dim, nh, nkv, 192, 256, 2, seed=7, group_ranks=gr, use_fused_k=fused)
    att = _drive(gpu, sd, palu, oracle, dim, nh, nkv, B, S0, steps, "tiled", fused)
    assert att.group_ranks == ([96, 192], [256, 64])
    assert all(isinstance(c, GroupedLatentCache) for c in att.layer_past)
    assert att.kv_bytes_per_token() == (96 + 192 + 256 + 64) * 2.0


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("rank_multiple,expect", [(32, ([128, 160], [192, 96])), (64, ([128, 192], [192, 96]))])
def test_attention_from_a_dump_with_group_ranks_off_the_kernel_grid(gpu, tmp_path, fused, rank_multiple, expect):
    """A G-LRD factor directory whose group ranks are not multiples of 32 (K 100 / 140, V 176 / 96, as a
    real dump's head_wise_ranks may be), written by save_palu_dir and read by load_palu_dir at two rank
    multiples: the layer rounds each group rank up to 32 (the widest group at the padded width), the
    factors being zero past each group's rank, and decodes on the fused and the naive path to the layer
    oracle built from the same loaded factors."""
    dim, nh, nkv, B, S0, steps = 1024, 8, 4, 2, 40, 4
    g = torch.Generator().manual_seed(31)
    W = {"q": torch.randn(nh * HD, dim, generator=g) * 0.02, "k": torch.randn(nkv * HD, dim, generator=g) * 0.02,
         "v": torch.randn(nkv * HD, dim, generator=g) * 0.02, "o": torch.randn(dim, nh * HD, generator=g) * 0.02}
    fac = compress.factor_layers({0: {"k": W["k"], "v": W["v"]}}, nkv, [[100, 140]], [[176, 96]])
    lr = convert.load_palu_dir(convert.save_palu_dir(tmp_path / "dump", fac), 1, nkv, HD, rank_multiple=rank_multiple)[0]
    assert lr.group_size == 2 and lr.group_ranks_k == [100, 140] and lr.group_ranks_v == [176, 96]
    sd = {"layers.0.attention.wq.weight": convert.reverse_permute(W["q"], nh, nh * HD, dim),
          "layers.0.attention.wo.weight": W["o"]}
    for name, t in convert.palu_layer_tensors(W, lr, nh, nkv, HD).items():
        sd[f"layers.0.attention.palu.{name}"] = t
    palu = convert.PaluConfig(rank_k=[lr.r_k], rank_v=[lr.r_v], cache_id="dump", group_size=lr.group_size,
                              runtime=convert.PaluRuntime(use_fused_k=fused, check=True),
                              group_ranks=[(lr.group_ranks_k, lr.group_ranks_v)])
    oracle = ref.PaluRefAttention(nh, nkv, HD, THETA, LLAMA3, W["q"], W["o"],
                                  ref.Factors(lr.k_VT, lr.k_U, lr.v_VT, lr.v_U))
    att = _drive(gpu, sd, palu, oracle, dim, nh, nkv, B, S0, steps, "tiled", fused)
    assert att.group_ranks == expect


def _drive(gpu, sd, palu, oracle, dim, nh, nkv, B, S0, steps, layout, fused):
    att = PaluAttention(gpu, None, _Args(dim, nh, nkv, 128, B, palu), sd, None, 0, cache_layout=layout)
    assert att.use_fused_k == (fused and att.recon_k)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(B, S0 + steps, dim, generator=g)
    exp_pre = oracle.forward(x[:, :S0], 0)
    out_pre = att.forward(x[:, :S0].to(gpu), mode="prefill", user_id=0)
    _close(out_pre, exp_pre, "prefill")
    for t in range(S0, S0 + steps):
        exp = oracle.forward(x[:, t:t + 1], t)[:, 0]
        out = att.forward(x[:, t].to(gpu), torch.full((B,), t, dtype=torch.int32, device=gpu), mode="decode")
        torch.cuda.synchronize()
        _close(out, exp, f"decode step {t}")
    return att


def test_attention_kv_bytes_per_token(gpu):
    sd, palu, _ = _layer(512, 4, 2, 64, 32, 1, seed=1)
    att = PaluAttention(gpu, None, _Args(512, 4, 2, 64, 1, palu), sd, None, 0)
    assert att.kv_bytes_per_token() == 2 * (64 + 32) * 2.0
