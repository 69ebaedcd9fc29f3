"""Pins of the CPU oracle (oracle/palu_oracle.py) against independent facts.

Each check is chosen so that a plausible slip in the oracle (a transposed pair rotation, a wrong
interleave, a dropped scale, an off-by-one causal bound, a wrong GQA mapping) fails it:
  * closed forms and properties the reference's own tests assert (tests/test_fused.py:8-115,
    tests/test_compress.py, tests/test_reference.py:17-35);
  * bit-level or near-bit-level agreement with transformers' LlamaRotaryEmbedding / LlamaAttention /
    apply_rotary_pos_emb, a library routine independent of the oracle;
  * brute-force scalar loops on tiny inputs.
A last group plants mistakes in copies of oracle functions and shows the pins catch them.
"""
import math

import pytest
import torch

from oracle import palu_oracle as ref

HD = 128
THETA = 500000.0
LLAMA3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}


def _hf_rotary(head_dim=HD, rope_scaling=LLAMA3, theta=THETA):
    transformers = pytest.importorskip("transformers")
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
    cfg = transformers.LlamaConfig(hidden_size=head_dim * 4, num_attention_heads=4, num_key_value_heads=2,
                                   head_dim=head_dim, rope_theta=theta, rope_scaling=rope_scaling,
                                   max_position_embeddings=131072)
    return LlamaRotaryEmbedding(cfg)


def _meta_cols(x):
    """HF head-dim order [x_0..x_{d/2-1}, y_0..y_{d/2-1}] -> Meta interleave [x_0, y_0, x_1, y_1, ...]."""
    h = x.shape[-1] // 2
    return torch.stack([x[..., :h], x[..., h:]], dim=-1).reshape(*x.shape[:-1], 2 * h)


# ------------------------------------------------------------------------------------------------
# Pair rotation, w_rot, chunk rule (ref tests/test_fused.py:8-30)

def test_pair_rotation_matrix_maps_pairs_to_minus_x1_x0():
    T = ref.rope_transformation_matrix(HD)
    x = torch.randn(5, HD)
    r = x @ T
    assert torch.equal(r[:, 0::2], -x[:, 1::2]) and torch.equal(r[:, 1::2], x[:, 0::2])
    assert torch.equal(T @ T, -torch.eye(HD))          # a quarter turn twice is a half turn


def test_w_rot_is_u_k_and_u_k_times_T():
    u_k = torch.randn(3, 64, HD)
    w = ref.w_rot_from_u_k(u_k)
    assert w.shape == (3, 64, 2 * HD) and torch.equal(w[..., :HD], u_k)
    lat = torch.randn(3, 7, 64)
    torch.testing.assert_close(lat @ w[..., HD:], (lat @ u_k) @ ref.rope_transformation_matrix(HD))


def test_chunk_size_known_answers():
    # ref tests/test_fused.py:28-30
    assert [ref.chunk_size(s) for s in (96, 256, 1024, 4096, 8192, 8192 + 32)] == [32, 256, 512, 512, 512, 32]
    assert ref.chunk_size(1) == 1 and ref.chunk_size(3 * 1024) == 512 and ref.chunk_size(48) == 16


# ------------------------------------------------------------------------------------------------
# RoPE frequencies and tables against transformers

def test_inv_freq_matches_transformers_llama3_and_plain():
    for scaling in (LLAMA3, None):
        hf = _hf_rotary(rope_scaling=scaling).inv_freq.float()
        ours = ref.inv_freq(HD, THETA, scaling)
        torch.testing.assert_close(ours, hf, rtol=2e-7, atol=0)
    # the llama3 bands: lowest frequencies slowed by the full factor, highest untouched
    plain, scaled = ref.inv_freq(HD, THETA, None), ref.inv_freq(HD, THETA, LLAMA3)
    assert torch.equal(scaled[0], plain[0])
    torch.testing.assert_close(scaled[-1], plain[-1] / 8.0)


def test_cos_sin_tables_are_hf_rotary_in_meta_order():
    S = 3000
    cos, sin = ref.cos_sin_tables(HD, S, THETA, LLAMA3)
    assert cos.shape == (S + 513, HD) and cos.dtype == torch.float32
    assert torch.equal(cos[:, 0::2], cos[:, 1::2]) and torch.equal(sin[:, 0::2], sin[:, 1::2])
    assert torch.equal(cos[0], torch.ones(HD)) and torch.equal(sin[0], torch.zeros(HD))
    rot = _hf_rotary()
    pos = torch.arange(S + 513)[None]
    hc, hs = rot(torch.zeros(1, 1, HD), pos)
    torch.testing.assert_close(cos, _meta_cols(hc[0]), rtol=0, atol=2e-6)
    torch.testing.assert_close(sin, _meta_cols(hs[0]), rtol=0, atol=2e-6)
    tab = ref.cs_table(cos, sin, S)
    assert tab.shape == (S, 2 * HD) and torch.equal(tab[:, :HD], cos[:S]) and torch.equal(tab[:, HD:], sin[:S])
    step = ref.rot_step_table(cos, sin, 128)
    assert step.shape == (32, 2 * HD) and torch.equal(step[5, :HD], cos[128]) and torch.equal(step[0], step[31])


def test_meta_rotation_equals_hf_rotate_half_after_reverse_permute():
    """meta_rotate on Meta-ordered columns == transformers' apply_rotary_pos_emb on HF-ordered ones."""
    pytest.importorskip("transformers")
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    S = 40
    cos, sin = ref.cos_sin_tables(HD, S, THETA, LLAMA3)
    rot = _hf_rotary()
    hc, hs = rot(torch.zeros(1, 1, HD), torch.arange(S)[None])
    x_hf = torch.randn(1, 1, S, HD)
    y_hf, _ = apply_rotary_pos_emb(x_hf, x_hf, hc, hs)
    y_meta = ref.meta_rotate(_meta_cols(x_hf[0, 0]), cos[:S], sin[:S])
    torch.testing.assert_close(y_meta, _meta_cols(y_hf[0, 0]), rtol=1e-5, atol=1e-5)


def test_reverse_permute_is_the_meta_interleave_of_hf_rows():
    n, d, dim = 3, 16, 5
    W = torch.randn(n * d, dim)
    M = ref.reverse_permute(W, n, n * d, dim)
    for h in range(n):
        for i in range(d // 2):
            assert torch.equal(M[h * d + 2 * i], W[h * d + i])
            assert torch.equal(M[h * d + 2 * i + 1], W[h * d + d // 2 + i])


def test_angle_addition_and_relative_rotation_identity():
    # ref tests/test_fused.py:52-73: the chunk-relative rotation the MI355X kernel uses rests on these
    cos, sin = ref.cos_sin_tables(HD, 2048, THETA, None)
    p = torch.arange(0, 700)
    for c in (32, 128, 512):
        torch.testing.assert_close(cos[p] * cos[c] - sin[p] * sin[c], cos[p + c], atol=2e-4, rtol=0)
        torch.testing.assert_close(sin[p] * cos[c] + cos[p] * sin[c], sin[p + c], atol=2e-4, rtol=0)
    T = ref.rope_transformation_matrix(HD)
    rot = lambda x, s: x * cos[s] + (x @ T) * sin[s]
    q, k = torch.randn(HD), torch.randn(HD)
    pq, s0, t = 1500, 1024, 37
    q_rel = rot(q, pq) * cos[s0] - (rot(q, pq) @ T) * sin[s0]
    torch.testing.assert_close(rot(q, pq) @ rot(k, s0 + t), q_rel @ rot(k, t), atol=1e-3, rtol=1e-5)


# ------------------------------------------------------------------------------------------------
# The op model

def _brute_attention(q, K, V, L, scale):
    """Scalar softmax attention of one query row over the first L rows (Python floats)."""
    s = [scale * float(q @ K[t]) for t in range(L)]
    m = max(s)
    e = [math.exp(x - m) for x in s]
    z = sum(e)
    return sum((e[t] / z) * V[t].double() for t in range(L))


def test_reference_decode_is_causal_gqa_attention_without_rotation():
    # ref tests/test_fused.py:76-89, with a scalar loop and an uneven GQA factor
    B, nkv, nh, S, r_v = 2, 2, 6, 24, 32
    q = torch.randn(1, B, nh, HD)
    k = torch.randn(B, nkv, S, HD)
    v = torch.randn(B, nkv, S, r_v)
    cur = torch.tensor([9, 23])
    out = ref.reference_decode(q, k, torch.eye(HD).expand(nkv, HD, HD), v, cur, torch.ones(S, HD),
                               torch.zeros(S, HD), 0.37)
    assert out.shape == (1, B, nh, r_v)
    for b in range(B):
        for h in range(nh):
            j = h // (nh // nkv)
            exp = _brute_attention(q[0, b, h], k[b, j], v[b, j], int(cur[b]) + 1, 0.37)
            torch.testing.assert_close(out[0, b, h].double(), exp, atol=1e-5, rtol=1e-4)


def test_reference_decode_scores_are_hf_rope_scores():
    """K rebuilt in Meta order and rotated by the tables == HF rotate_half RoPE on HF-ordered u_k."""
    pytest.importorskip("transformers")
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    S, r_k, r_v, nh = 50, 32, 16, 2
    lat = torch.randn(1, 1, S, r_k)
    u_hf = torch.randn(1, r_k, HD) * 0.2                   # HF head order columns
    v = torch.randn(1, 1, S, r_v)
    q_hf = torch.randn(nh, HD)
    pos = S - 1
    rot = _hf_rotary()
    hc, hs = rot(torch.zeros(1, 1, HD), torch.arange(S)[None])
    K_hf = (lat[0, 0] @ u_hf[0])[None, None]
    K_hf, _ = apply_rotary_pos_emb(K_hf, K_hf, hc, hs)
    qr, _ = apply_rotary_pos_emb(q_hf[None, :, None], q_hf[None, :, None], hc[:, pos:pos + 1], hs[:, pos:pos + 1])
    qr = qr[0, :, 0]                                        # [nh, HD], rotated at its own position
    exp = torch.softmax(qr @ K_hf[0, 0].T * HD ** -0.5, -1) @ v[0, 0]
    cos, sin = ref.cos_sin_tables(HD, S, THETA, LLAMA3)
    out = ref.reference_decode(_meta_cols(qr)[None, None], lat, _meta_cols(u_hf), v, torch.tensor([pos]),
                               cos, sin, HD ** -0.5)
    torch.testing.assert_close(out[0, 0], exp, atol=1e-5, rtol=1e-4)


def test_reference_decode_u_v_mode_equals_prebuilt_v():
    # ref tests/test_fused.py:106-115, with grouped latents (2 KV heads share one latent head)
    B, nlat, nkv, nh, S, r_k, r_v = 1, 1, 2, 4, 16, 32, 48
    q = torch.randn(1, B, nh, HD)
    k = torch.randn(B, nlat, S, r_k)
    u_k = torch.randn(nkv, r_k, HD)
    v_lat = torch.randn(B, nlat, S, r_v)
    u_v = torch.randn(nkv, r_v, HD)
    cos, sin = ref.cos_sin_tables(HD, S, THETA, None)
    cur = torch.tensor([S - 3])
    out = ref.reference_decode(q, k, u_k, v_lat, cur, cos, sin, 0.1, u_v=u_v)
    v_full = torch.einsum("bsr,hrd->bhsd", v_lat[:, 0], u_v)
    k_rep = k.repeat_interleave(nkv, dim=1)
    exp = ref.reference_decode(q, k_rep, u_k, v_full, cur, cos, sin, 0.1)
    assert out.shape == (1, B, nh, HD)
    torch.testing.assert_close(out, exp, atol=1e-5, rtol=1e-4)


def test_full_kv_decode_brute_force():
    B, nkv, nh, S, dv = 1, 2, 4, 12, 8
    q, k, v = torch.randn(1, B, nh, HD), torch.randn(B, nkv, S, HD), torch.randn(B, nkv, S, dv)
    out = ref.full_kv_decode(q, k, v, torch.tensor([7]), 0.2)
    for h in range(nh):
        exp = _brute_attention(q[0, 0, h], k[0, h // 2], v[0, h // 2], 8, 0.2)
        torch.testing.assert_close(out[0, 0, h].double(), exp, atol=1e-5, rtol=1e-4)


# ------------------------------------------------------------------------------------------------
# Layer oracle against transformers (ref tests/test_reference.py:17-35)

def _small_layer(seed=0, hidden=256, nh=4, nkv=2, hd=64):
    g = torch.Generator().manual_seed(seed)
    W = {n: torch.randn(o, hidden, generator=g) * 0.05
         for n, o in (("q", nh * hd), ("k", nkv * hd), ("v", nkv * hd), ("o", hidden))}
    W["o"] = torch.randn(hidden, nh * hd, generator=g) * 0.05
    return W


def test_identity_factor_layer_equals_transformers_llama_attention():
    transformers = pytest.importorskip("transformers")
    from transformers.models.llama.modeling_llama import LlamaAttention, LlamaRotaryEmbedding
    hidden, nh, nkv, hd, S = 256, 4, 2, 64, 19
    cfg = transformers.LlamaConfig(hidden_size=hidden, num_attention_heads=nh, num_key_value_heads=nkv, head_dim=hd,
                                   rope_theta=THETA, rope_scaling=LLAMA3, max_position_embeddings=131072,
                                   attention_bias=False)
    cfg._attn_implementation = "eager"
    W = _small_layer(hidden=hidden, nh=nh, nkv=nkv, hd=hd)
    att = LlamaAttention(cfg, layer_idx=0).eval()
    with torch.no_grad():
        att.q_proj.weight.copy_(W["q"]); att.k_proj.weight.copy_(W["k"])
        att.v_proj.weight.copy_(W["v"]); att.o_proj.weight.copy_(W["o"])
    x = torch.randn(1, S, hidden)
    pe = LlamaRotaryEmbedding(cfg)(x, torch.arange(S)[None])
    mask = torch.full((S, S), float("-inf")).triu(1)[None, None]
    with torch.no_grad():
        exp, _ = att(x, position_embeddings=pe, attention_mask=mask)
    seen = {}
    att.o_proj.register_forward_pre_hook(lambda mod, args: seen.setdefault("attn", args[0].detach().clone()))
    with torch.no_grad():
        att(x, position_embeddings=pe, attention_mask=mask)
    layer = ref.PaluRefAttention(nh, nkv, hd, THETA, LLAMA3, W["q"], W["o"], ref.identity_factors(W["k"], W["v"], nkv, hd))
    out = layer.forward(x, 0)
    torch.testing.assert_close(out, exp, atol=1e-4, rtol=1e-4)
    # the attention output before o_proj (what the fused op computes, in head space) equals transformers'
    # o_proj input, and o_proj of it is the layer output
    layer2 = ref.PaluRefAttention(nh, nkv, hd, THETA, LLAMA3, W["q"], W["o"], ref.identity_factors(W["k"], W["v"], nkv, hd))
    out2, attn = layer2.forward(x, 0, return_attention=True)
    torch.testing.assert_close(attn, seen["attn"].reshape(attn.shape), atol=1e-5, rtol=1e-4)
    torch.testing.assert_close(out2, attn @ W["o"].float().T, atol=0, rtol=0)


def _tiny_llama_weights(cfg, seed):
    g = torch.Generator().manual_seed(seed)
    d, f, hd, nh, nkv, V = cfg["dim"], cfg["ffn_dim"], cfg["head_dim"], cfg["n_heads"], cfg["n_kv_heads"], cfg["vocab_size"]
    r = lambda *s: torch.randn(*s, generator=g) * 0.05
    w = {"model.embed_tokens.weight": r(V, d), "model.norm.weight": 1 + r(d), "lm_head.weight": r(V, d)}
    dense = []
    for i in range(cfg["n_layers"]):
        p = f"model.layers.{i}."
        w.update({p + "self_attn.q_proj.weight": r(nh * hd, d), p + "self_attn.o_proj.weight": r(d, nh * hd),
                  p + "mlp.gate_proj.weight": r(f, d), p + "mlp.up_proj.weight": r(f, d), p + "mlp.down_proj.weight": r(d, f),
                  p + "input_layernorm.weight": 1 + r(d), p + "post_attention_layernorm.weight": 1 + r(d)})
        dense.append((r(nkv * hd, d), r(nkv * hd, d)))
    return w, dense


_TINY = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, vocab_size=97, ffn_dim=384, norm_eps=1e-5,
             rope_theta=THETA, rope_scaling=LLAMA3)


def test_lowrank_proj_is_the_dense_factor_product():
    g = torch.Generator().manual_seed(5)
    VT, U = torch.randn(3, 8, 40, generator=g), torch.randn(3, 16, 8, generator=g)
    x = torch.randn(2, 7, 40, generator=g)
    dense = torch.cat([U[h] @ VT[h] for h in range(3)])                  # [3 * 16, 40]
    torch.testing.assert_close(ref.LowRankProj(VT, U)(x), x @ dense.T, atol=1e-4, rtol=1e-4)


def test_lowrank_llama_full_rank_equals_transformers_dense_model():
    transformers = pytest.importorskip("transformers")
    w, dense = _tiny_llama_weights(_TINY, seed=3)
    nkv, hd = _TINY["n_kv_heads"], _TINY["head_dim"]
    model = ref.lowrank_llama(_TINY, w, [ref.identity_factors(k, v, nkv, hd) for k, v in dense])
    m2 = ref.lowrank_llama(_TINY, w, [ref.identity_factors(k, v, nkv, hd) for k, v in dense])
    for i, (k, v) in enumerate(dense):                    # back to plain dense projections
        att = m2.model.layers[i].self_attn
        att.k_proj = torch.nn.Linear(_TINY["dim"], nkv * hd, bias=False)
        att.v_proj = torch.nn.Linear(_TINY["dim"], nkv * hd, bias=False)
        with torch.no_grad():
            att.k_proj.weight.copy_(k); att.v_proj.weight.copy_(v)
    ids = torch.randint(0, _TINY["vocab_size"], (2, 21), generator=torch.Generator().manual_seed(0))
    with torch.no_grad():
        a, b = model(ids).logits, m2(ids).logits
    torch.testing.assert_close(a, b, atol=1e-4, rtol=1e-4)
    assert isinstance(m2, transformers.LlamaForCausalLM)


def test_lowrank_llama_attention_is_the_layer_oracle():
    """The low-rank model's attention sublayer (inputs captured by a hook) equals PaluRefAttention with
    the same truncated factors: ties the model-level oracle to the layer oracle."""
    pytest.importorskip("transformers")
    cfg = dict(_TINY, n_layers=1)
    w, dense = _tiny_llama_weights(cfg, seed=4)
    nkv, hd, nh = cfg["n_kv_heads"], cfg["head_dim"], cfg["n_heads"]
    Uk, VTk = ref.svd_per_head(dense[0][0], nkv, 24)
    Uv, VTv = ref.svd_per_head(dense[0][1], nkv, 40)
    f = ref.Factors(VTk, Uk, VTv, Uv)
    model = ref.lowrank_llama(cfg, w, [f])
    seen = {}
    att = model.model.layers[0].self_attn
    att.register_forward_hook(lambda m, a, kw, out: seen.update(x=kw["hidden_states"], y=out[0]), with_kwargs=True)
    ids = torch.randint(0, cfg["vocab_size"], (1, 17), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        model(ids)
    layer = ref.PaluRefAttention(nh, nkv, hd, THETA, LLAMA3, w["model.layers.0.self_attn.q_proj.weight"],
                                 w["model.layers.0.self_attn.o_proj.weight"], f)
    torch.testing.assert_close(layer.forward(seen["x"], 0), seen["y"], atol=1e-4, rtol=1e-4)


def test_layer_prefill_then_decode_equals_fresh_prefill():
    hidden, nh, nkv, hd = 256, 4, 2, 64
    W = _small_layer(seed=1)
    Uk, VTk = ref.svd_per_head(W["k"], nkv, 16)
    Uv, VTv = ref.svd_per_head(W["v"], nkv, 16)
    f = ref.Factors(VTk, Uk, VTv, Uv)
    x = torch.randn(1, 12, hidden)
    a = ref.PaluRefAttention(nh, nkv, hd, THETA, LLAMA3, W["q"], W["o"], f)
    full = a.forward(x, 0)
    b = ref.PaluRefAttention(nh, nkv, hd, THETA, LLAMA3, W["q"], W["o"], f)
    b.forward(x[:, :8], 0)
    steps = [b.forward(x[:, t:t + 1], t) for t in range(8, 12)]
    torch.testing.assert_close(torch.cat(steps, dim=1), full[:, 8:], atol=1e-5, rtol=1e-4)


def test_op_model_equals_layer_oracle_decode_attention():
    """The fused-op model on the converted factors (u_k = reverse_permute(k_U)^T, Meta-order q) gives the
    same attention as the HF-convention layer oracle, before o_proj."""
    hidden, nh, nkv, hd, rank, T = 256, 4, 2, 64, 32, 10
    W = _small_layer(seed=2)
    Uk, VTk = ref.svd_per_head(W["k"], nkv, rank)
    Uv, VTv = ref.svd_per_head(W["v"], nkv, rank)
    x = torch.randn(1, T, hidden)
    layer = ref.PaluRefAttention(nh, nkv, hd, THETA, LLAMA3, W["q"], torch.eye(hidden, nh * hd), ref.Factors(VTk, Uk, VTv, Uv))
    layer.forward(x[:, :-1], 0)
    exp = layer.forward(x[:, -1:], T - 1)[0, 0].view(nh, hd)
    # op inputs: latents, Meta-order u_k, absorbed V rebuilt with u_v = v_U^T, q rotated at T-1 in Meta order
    k_lat = torch.einsum("bsd,hrd->bhsr", x, VTk)
    v_lat = torch.einsum("bsd,hrd->bhsr", x, VTv)
    u_k = torch.stack([ref.reverse_permute(Uk[h], 1, hd, rank).T for h in range(nkv)])
    u_v = Uv.transpose(1, 2)
    cq, sq = ref.hf_cos_sin(torch.tensor([T - 1]), hd, THETA, LLAMA3)
    q = (x[:, -1] @ W["q"].T).view(nh, hd)
    q = q * cq + ref.rotate_half(q) * sq
    q_meta = torch.stack([ref.reverse_permute(q[h][:, None], 1, hd, 1)[:, 0] for h in range(nh)])
    cos, sin = ref.cos_sin_tables(hd, T, THETA, LLAMA3)
    out = ref.reference_decode(q_meta[None, None], k_lat, u_k, v_lat, torch.tensor([T - 1]), cos, sin,
                               hd ** -0.5, u_v=u_v)
    torch.testing.assert_close(out[0, 0], exp, atol=1e-5, rtol=1e-4)


# ------------------------------------------------------------------------------------------------
# Factor production (ref tests/test_compress.py)

def test_svd_per_head_exact_at_full_rank_and_balanced():
    W = torch.randn(2 * 16, 40)
    U, VT = ref.svd_per_head(W, 2, 16)
    torch.testing.assert_close(U @ VT, W.view(2, 16, 40), atol=1e-4, rtol=1e-4)
    for h in range(2):     # balanced split: U^T U == VT VT^T == diag(sigma)
        torch.testing.assert_close(U[h].T @ U[h], VT[h] @ VT[h].T, atol=1e-4, rtol=1e-4)
    errs = []
    for r in (2, 4, 8, 12):
        U, VT = ref.svd_per_head(W, 2, r)
        errs.append(float((U @ VT - W.view(2, 16, 40)).norm()))
    assert errs == sorted(errs, reverse=True) and errs[0] > errs[-1]


# ------------------------------------------------------------------------------------------------
# Planted mistakes: copies of oracle pieces with one plausible slip each must fail the pins above.

def test_pins_catch_planted_mistakes():
    S = 30
    cos, sin = ref.cos_sin_tables(HD, S, THETA, LLAMA3)
    rot = _hf_rotary()
    hc, hs = rot(torch.zeros(1, 1, HD), torch.arange(S + 513)[None])
    # (1) sin sign flipped in the rotation -> differs from HF RoPE
    x = torch.randn(S, HD)
    good = ref.meta_rotate(x, cos[:S], sin[:S])
    bad = ref.meta_rotate(x, cos[:S], -sin[:S])
    assert not torch.allclose(good, bad, atol=1e-3)
    # (2) tables in HF half-split order instead of Meta interleave -> fail the interleave/HF check
    assert not torch.allclose(hc[0], _meta_cols(hc[0]), atol=1e-3)
    # (3) off-by-one causal bound (attending cur_pos + 2 rows) -> differs from the brute force
    q, k, v = torch.randn(1, 1, 2, HD), torch.randn(1, 1, 8, HD), torch.randn(1, 1, 8, 4)
    eye, ones, zeros = torch.eye(HD)[None], torch.ones(8, HD), torch.zeros(8, HD)
    a = ref.reference_decode(q, k, eye, v, torch.tensor([4]), ones, zeros, 0.3)
    b = ref.reference_decode(q, k, eye, v, torch.tensor([5]), ones, zeros, 0.3)
    assert not torch.allclose(a, b, atol=1e-4)
    # (4) plain frequencies where llama3 scaling is asked for -> differ from transformers' llama3 values
    assert not torch.allclose(ref.inv_freq(HD, THETA, None), rot.inv_freq.float(), rtol=1e-3)


def test_gather_pages_follows_the_page_table_position_by_position():
    G, ps, r, B, maxp = 2, 4, 3, 3, 5
    pool = torch.randn(11, G, ps, r)
    pt = torch.randint(0, 11, (B, maxp), dtype=torch.int32)
    rows = ref.gather_pages(pool, pt)
    assert rows.shape == (B, G, maxp * ps, r)
    for b in range(B):
        for g in range(G):
            for p in range(maxp * ps):
                assert torch.equal(rows[b, g, p], pool[int(pt[b, p // ps]), g, p % ps])


# ------------------------------------------------------------------------------------------------
# The comparison metrics every parity verdict uses

def test_metric_helpers_match_library_routines():
    """pcc, cosine and max_abs against torch.corrcoef, F.cosine_similarity and the plain max abs
    difference on random inputs of several shapes and scales; a constant offset changes the cosine but
    not the PCC (PCC centres both inputs, cosine does not), and a single changed element moves max_abs
    by exactly its change."""
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(11)
    for shape, scale in (((1000,), 1.0), ((7, 33), 1e-3), ((2, 3, 64), 50.0)):
        a = torch.randn(*shape, generator=g) * scale
        b = a + 0.3 * scale * torch.randn(*shape, generator=g)
        exp_pcc = float(torch.corrcoef(torch.stack([a.flatten().double(), b.flatten().double()]))[0, 1])
        exp_cos = float(F.cosine_similarity(a.flatten().double(), b.flatten().double(), dim=0))
        assert abs(ref.pcc(a, b) - exp_pcc) < 1e-12
        assert abs(ref.cosine(a, b) - exp_cos) < 1e-12
        assert ref.max_abs(a, b) == float((a.double() - b.double()).abs().max())
        off = b + 5.0 * scale
        assert abs(ref.pcc(a, off) - ref.pcc(a, b)) < 1e-6       # the fp32 sum b + offset rounds b
        assert ref.cosine(a, off) < ref.cosine(a, b) - 1e-3
    x = torch.zeros(50)
    y = x.clone()
    y[17] = -0.25
    assert ref.max_abs(x, y) == 0.25 and ref.max_abs(y, x) == 0.25
    assert ref.cosine(x, x) == 1.0 and ref.pcc(x, x) == 1.0          # zero inputs: equal -> 1
    assert ref.cosine(x, y) == 0.0
    z = torch.randn(64, generator=g)
    assert ref.pcc(z, -z) == pytest.approx(-1.0, abs=1e-12) and ref.cosine(z, 2 * z) == pytest.approx(1.0, abs=1e-12)
