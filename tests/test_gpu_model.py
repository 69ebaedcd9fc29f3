"""End-to-end decoder (palu_tt.model.Transformer) against the fp32 low-rank Llama oracle, teacher-forced,
as the reference's decode-fidelity harness compares models (palu_tt/decode_check.py:47-133: one prefill,
then decode steps fed the same next tokens, PCC per step).

The model is random-init with per-layer ranks that exercise every attention path at once: fused latent
decode (r < head_dim), the full-rank K fast path and the stock full-KV path (r_k = r_v = head_dim), and
rank padding to a multiple of 32. The oracle is transformers' LlamaForCausalLM in fp32 with k_proj / v_proj
computed through the same factors (oracle.lowrank_llama), run once over prompt + teacher tokens. The GPU
model runs in bf16, so the bar is on logits: PCC >= 0.999 per step and max-abs within 3% of the largest
logit magnitude. The HIP-graph decode step must reproduce the eager step.
"""
import pytest
import torch

from oracle import palu_oracle as ref
from palu_tt import model as pm

pytestmark = pytest.mark.gpu


def _hf_weights(sd, dense, n_layers):
    """HF-named fp32 weights of the bf16 model (q_proj back in HF head order from the dense copy)."""
    f = lambda k: sd[k].float().cpu()
    w = {"model.embed_tokens.weight": f("tok_embeddings.weight"), "model.norm.weight": f("norm.weight"),
         "lm_head.weight": f("output.weight")}
    for i in range(n_layers):
        p, q = f"layers.{i}.", f"model.layers.{i}."
        w[q + "self_attn.q_proj.weight"] = dense[i][0]["q"].to(torch.bfloat16).float()
        w[q + "self_attn.o_proj.weight"] = f(p + "attention.wo.weight")
        w[q + "mlp.gate_proj.weight"] = f(p + "feed_forward.w1.weight")
        w[q + "mlp.up_proj.weight"] = f(p + "feed_forward.w3.weight")
        w[q + "mlp.down_proj.weight"] = f(p + "feed_forward.w2.weight")
        w[q + "input_layernorm.weight"] = f(p + "attention_norm.weight")
        w[q + "post_attention_layernorm.weight"] = f(p + "ffn_norm.weight")
    return w


def _check(out, exp, what):
    out, exp = out.float().cpu(), exp.float()
    for b in range(out.shape[0]):
        p = ref.pcc(out[b], exp[b])
        rel = ref.max_abs(out[b], exp[b]) / float(exp[b].abs().max())
        assert p >= 0.999 and rel <= 0.03, f"{what} row {b}: pcc {p:.6f}, max-abs / max {rel:.4f}"


@pytest.mark.parametrize("layout,vocab", [("tiled", 1024), ("rows", 1024), ("tiled", 1000)])
def test_decoder_teacher_forced_matches_lowrank_llama(gpu, layout, vocab):
    """vocab 1024: every decode projection tiled, so the step is the fused one (QKV epilogue in the
    projection, residual add in the output projection, FFN norm folded into gate / up); vocab 1000: the
    LM head is not a multiple of 16 columns, so the step runs its separate norms over row-major
    activations (with the gate / up weight still folded). The norms' weights are drawn around 1, so the
    folding is exercised."""
    pytest.importorskip("transformers")
    args = pm.ModelArgs(dim=512, n_layers=3, n_heads=4, n_kv_heads=2, vocab_size=vocab, ffn_dim=1024,
                        max_seq_len=128, max_batch_size=2)
    dense = []
    sd = pm.random_palu_state_dict(args, [40, 64, 128], [32, 128, 72], gpu, seed=11, std=0.05, dense_out=dense)
    gn = torch.Generator().manual_seed(12)
    for key in [k for k in sd if k.endswith("_norm.weight") or k == "norm.weight"]:
        sd[key] = (1 + 0.2 * torch.randn(args.dim, generator=gn)).to(sd[key].device, sd[key].dtype)
    assert args.palu.rank_k == [64, 64, 128] and args.palu.rank_v == [32, 128, 96]
    hf_w = _hf_weights(sd, dense, args.n_layers)
    cfg = dict(dim=args.dim, n_layers=args.n_layers, n_heads=args.n_heads, n_kv_heads=args.n_kv_heads,
               head_dim=args.head_dim, vocab_size=args.vocab_size, ffn_dim=args.ffn_dim, norm_eps=args.norm_eps,
               rope_theta=args.rope_theta, rope_scaling=args.rope_scaling)
    oracle = ref.lowrank_llama(cfg, hf_w, [ref.Factors(lr.k_VT, lr.k_U, lr.v_VT, lr.v_U) for _, lr in dense])
    model = pm.Transformer(args, sd, gpu, cache_layout=layout)
    assert model._fused_step == (vocab % 16 == 0)
    assert all(L["w13"].in_scale_folded for L in model.layers)

    B, S, steps = 2, 45, 7
    g = torch.Generator().manual_seed(2)
    ids = torch.randint(0, args.vocab_size, (B, S + steps), generator=g)
    with torch.no_grad():
        exp = oracle(ids).logits                                          # [B, S + steps, vocab]
    _check(pm.prefill_all(model, ids[:, :S].to(gpu), users_per_chunk=1), exp[:, S - 1], "prefill")
    for t in range(steps):
        tok = ids[:, S + t].to(gpu)
        pos = torch.full((B,), S + t, dtype=torch.int32, device=gpu)
        eager = model.decode(tok, pos)
        graph = model.decode_graph(tok, pos).clone()                      # rewrites the same cache rows
        greedy = model.decode_graph(tok, pos, greedy=True).clone()
        torch.cuda.synchronize()
        _check(eager, exp[:, S + t], f"decode step {t}")
        assert ref.cosine(graph.cpu(), eager.cpu()) >= 0.99999, f"graph replay differs at step {t}"
        # the greedy graph's ids pick a maximal logit of the step (up to the steps' own differences)
        e = eager.cpu()
        assert (e.max(-1).values - e.gather(1, greedy.cpu()[:, None])[:, 0]).abs().max() <= 1e-2 * e.abs().max()


def test_decoder_above_64_rows_matches_lowrank_llama(gpu):
    """Past 64 rows the decode projections are torch's F.linear and the step keeps its separate norms
    (no tiled activations, no folded FFN norm): the same oracle bar, two teacher-forced steps."""
    pytest.importorskip("transformers")
    args = pm.ModelArgs(dim=512, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=700, ffn_dim=1024,
                        max_seq_len=64, max_batch_size=65)
    dense = []
    sd = pm.random_palu_state_dict(args, [64, 48], [32, 96], gpu, seed=13, std=0.05, dense_out=dense)
    hf_w = _hf_weights(sd, dense, args.n_layers)
    cfg = dict(dim=args.dim, n_layers=args.n_layers, n_heads=args.n_heads, n_kv_heads=args.n_kv_heads,
               head_dim=args.head_dim, vocab_size=args.vocab_size, ffn_dim=args.ffn_dim, norm_eps=args.norm_eps,
               rope_theta=args.rope_theta, rope_scaling=args.rope_scaling)
    oracle = ref.lowrank_llama(cfg, hf_w, [ref.Factors(lr.k_VT, lr.k_U, lr.v_VT, lr.v_U) for _, lr in dense])
    model = pm.Transformer(args, sd, gpu)
    assert not model._fused_step and not any(L["w13"].in_scale_folded for L in model.layers)
    B, S, steps = 65, 20, 2
    ids = torch.randint(0, args.vocab_size, (B, S + steps), generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        exp = oracle(ids).logits
    pm.prefill_all(model, ids[:, :S].to(gpu), users_per_chunk=65)
    for t in range(steps):
        pos = torch.full((B,), S + t, dtype=torch.int32, device=gpu)
        out = model.decode(ids[:, S + t].to(gpu), pos)
        torch.cuda.synchronize()
        _check(out, exp[:, S + t], f"decode step {t}")


def test_generate_greedy_is_consistent_with_decode(gpu):
    """generate() (graph decode) returns, at every step, the argmax of the eager decode's logits for the
    tokens it generated (teacher-forced replay on a fresh model built from the same seed)."""
    mk = lambda: pm.ModelArgs(dim=512, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=512, ffn_dim=768,
                              max_seq_len=96, max_batch_size=3)
    a1 = mk()
    m1 = pm.Transformer(a1, pm.random_palu_state_dict(a1, [48, 96], [64, 32], gpu, seed=5, std=0.1), gpu)
    prompts = torch.randint(0, 512, (3, 33), generator=torch.Generator().manual_seed(8)).to(gpu)
    out = pm.generate(m1, prompts, n_new=6)
    assert out.shape == (3, 6)
    a2 = mk()
    m2 = pm.Transformer(a2, pm.random_palu_state_dict(a2, [48, 96], [64, 32], gpu, seed=5, std=0.1), gpu)
    logits = pm.prefill_all(m2, prompts)
    margins = []
    for t in range(6):
        top2 = logits.topk(2, dim=-1).values
        margins.append(top2[:, 0] - top2[:, 1])
        close = margins[-1] < 1e-2 * top2[:, 0].abs().clamp_min(1.0)       # near-ties may flip in bf16
        assert torch.all((logits.argmax(-1) == out[:, t]) | close), f"step {t}"
        if t < 5:
            logits = m2.decode(out[:, t], torch.full((3,), 33 + t, dtype=torch.int32, device=gpu))


def test_deterministic_decode_is_bit_reproducible(gpu):
    """PaluRuntime.deterministic (Transformer.set_deterministic, generate(..., deterministic=True)) fixes the
    decode kernels' block order: the same decode step repeated from the same state gives the same logits
    bit for bit, eager and from the HIP graph, the greedy step's ids (picked inside the LM head) are the
    argmax of those logits, and greedy generation gives the same ids on every run."""
    args = pm.ModelArgs(dim=512, n_layers=2, n_heads=8, n_kv_heads=2, vocab_size=640, ffn_dim=1024,
                        max_seq_len=640, max_batch_size=4)
    model = pm.Transformer(args, pm.random_palu_state_dict(args, [64, 96], [48, 64], gpu, seed=21, std=0.1), gpu)
    model.set_deterministic(True)
    prompts = torch.randint(0, args.vocab_size, (4, 500), generator=torch.Generator().manual_seed(22)).to(gpu)
    first = pm.prefill_all(model, prompts).argmax(-1)
    pos = torch.full((4,), 500, dtype=torch.int32, device=gpu)
    a = model.decode(first, pos).clone()          # the step rewrites the same cache position each time
    b = model.decode(first, pos).clone()
    c = model.decode_graph(first, pos).clone()
    d = model.decode_graph(first, pos).clone()
    ge = model.decode(first, pos, greedy=True).clone()      # the pick fused into the LM head
    gg = model.decode_graph(first, pos, greedy=True).clone()
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(c, d) and torch.equal(a, c)
    assert model._fused_step and model.output.tiled
    want = torch.argmax(a.cpu(), dim=-1)                   # argmax of the same step's bf16 logits
    assert torch.equal(ge.cpu(), want) and torch.equal(gg.cpu(), want)
    g1 = pm.generate(model, prompts, n_new=8, deterministic=True)
    g2 = pm.generate(model, prompts, n_new=8, deterministic=True)
    assert torch.equal(g1, g2)
