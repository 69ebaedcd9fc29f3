"""A Llama-3.1-shaped decoder whose attention layers are PaluAttention (latent caches, fused latent
decode on MI355X): the end-to-end path of the reference's palu_tt/model.py + generate.py:53-62 and
decode_check.py:47-133, on PyTorch-ROCm.

Weights follow the tt_transformers state-dict names the reference loads (tok_embeddings, layers.{i}.
attention_norm / attention.wq|wk|wv|wo / ffn_norm / feed_forward.w1|w2|w3, norm, output) plus the
converter's layers.{i}.attention.palu.*. ``random_palu_state_dict`` builds a random-init model with
per-layer M-LRD ranks (per-head SVD of random k/v projections, ranks padded up to a multiple of 32 as
convert.load_palu_dir does, or V ranks to a multiple of 16 for tiled caches), which is what the
end-to-end benchmark uses.

Decode runs every projection on the library's M <= 64 projection kernel over weights held tiled
(decoder_ops.DecodeLinear), and the attention core and the elementwise work around it (RMSNorm with the
residual add, RoPE and the latent appends fused into one QKV epilogue, SwiGLU in the gate/up epilogue)
through the HIP library; ``Transformer.decode_graph`` captures a whole decode step in a HIP graph so a
step is one graph launch.
"""
import math
from dataclasses import dataclass, field
from typing import List, Optional

import torch
import torch.nn.functional as F

from palu_tt import compress, convert, decoder_ops
from palu_tt.attention import PaluAttention

LLAMA3_SCALING = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                  "original_max_position_embeddings": 8192}


@dataclass
class ModelArgs:
    dim: int = 4096
    n_layers: int = 32
    n_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 128
    vocab_size: int = 128256
    ffn_dim: int = 14336
    norm_eps: float = 1e-5
    rope_theta: float = 500000.0
    rope_scaling: Optional[dict] = field(default_factory=lambda: dict(LLAMA3_SCALING))
    max_seq_len: int = 2304
    max_batch_size: int = 1
    palu: Optional[convert.PaluConfig] = None


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()).to(x.dtype)


class Transformer(torch.nn.Module):
    def __init__(self, args: ModelArgs, state_dict: dict, device, cache_layout: str = "tiled"):
        super().__init__()
        assert args.palu is not None, "ModelArgs.palu must hold the per-layer ranks (a PaluConfig)"
        self.args = args
        self.device = torch.device(device)
        bf, dev = torch.bfloat16, self.device
        t = lambda k: state_dict.pop(k).to(dev, bf)
        self.tok_embeddings = t("tok_embeddings.weight")
        self.norm_w = t("norm.weight")
        # projections of the decode step, held in its tiled order (decoder_ops.DecodeLinear); the prefill
        # multiplies by nn.Linear-layout copies made per call
        rows = args.max_batch_size
        self.output = decoder_ops.DecodeLinear(t("output.weight"), rows)         # [vocab, dim]
        self.layers = []
        for i in range(args.n_layers):
            p = f"layers.{i}"
            attn_sd = {k: v for k, v in state_dict.items() if k.startswith(f"{p}.attention.")}
            attn = PaluAttention(dev, None, args, attn_sd, None, i, cache_layout=cache_layout)
            for k in attn_sd:
                state_dict.pop(k)
            # the FFN norm's weight is folded into a tiled gate / up weight (then the norm in front of it
            # multiplies by ones, and the decode step normalises inside the gate / up launch)
            ffn_norm = t(f"{p}.ffn_norm.weight")
            w13 = decoder_ops.DecodeLinear(None, rows, gate_up=(t(f"{p}.feed_forward.w1.weight"),
                                                                t(f"{p}.feed_forward.w3.weight")), in_scale=ffn_norm)
            if w13.in_scale_folded:
                ffn_norm = torch.ones_like(ffn_norm)
            self.layers.append(dict(attn=attn, attn_norm=t(f"{p}.attention_norm.weight"), ffn_norm=ffn_norm, w13=w13,
                                    w2=decoder_ops.DecodeLinear(t(f"{p}.feed_forward.w2.weight"), rows)))
        # tiled activations between the decode step's kernels where every projection that reads them is tiled
        self._tiled_acts = self.output.tiled and all(
            L["w13"].tiled and L["w2"].tiled and L["attn"].wqkv.tiled for L in self.layers)
        # the fused step: output projections add into the residual stream, the FFN norm runs inside gate / up
        self._fused_step = self._tiled_acts and all(
            L["w13"].in_scale_folded and L["attn"].wo_out.tiled and L["attn"].wo_out.ks == 1 for L in self.layers)
        self._graph = None

    def set_deterministic(self, deterministic: bool) -> None:
        """PaluRuntime.deterministic for every layer (a fixed block order in the decode kernels, so repeated
        decodes are bit-identical); a captured decode graph is dropped."""
        self.args.palu.runtime.deterministic = bool(deterministic)
        self._graph = None

    def set_fused_k(self, use_fused_k: bool, recon_len: Optional[int] = None) -> None:
        """Switches every layer between the fused latent decode and the naive path (PaluRuntime.use_fused_k,
        recon_len), as the reference selects per built model; a captured decode graph is dropped."""
        self.args.palu.runtime.use_fused_k = bool(use_fused_k)
        self.args.palu.runtime.recon_len = recon_len
        for L in self.layers:
            att = L["attn"]
            att.use_fused_k = att.recon_k and bool(use_fused_k)
        self._graph = None

    def _ffn(self, L, h):
        gu = F.linear(h, L["w13"].plain())
        g, u = gu.chunk(2, dim=-1)
        return F.linear((F.silu(g.float()) * u.float()).to(h.dtype), L["w2"].plain())

    @torch.no_grad()
    def prefill(self, tokens: torch.Tensor, user_id: int = 0) -> torch.Tensor:
        """tokens [U, S] for cache rows user_id .. user_id + U - 1 (positions 0 .. S-1); returns the
        logits of the last position of every row, [U, vocab]."""
        eps = self.args.norm_eps
        h = self.tok_embeddings[tokens]                                  # [U, S, dim]
        for L in self.layers:
            h = h + L["attn"].forward_prefill(rms_norm(h, L["attn_norm"], eps), user_id=user_id)
            h = h + self._ffn(L, rms_norm(h, L["ffn_norm"], eps))
        return F.linear(rms_norm(h[:, -1], self.norm_w, eps), self.output.plain()).float()

    @torch.no_grad()
    def decode(self, tokens: torch.Tensor, current_pos: torch.Tensor, greedy: bool = False) -> torch.Tensor:
        """One decode step for all max_batch_size rows: tokens [B] at positions current_pos [B] (int32,
        device); returns logits [B, vocab] fp32, or with greedy the argmax token ids [B] int64 taken from
        the bf16 logits (the same ids as argmax of the fp32 ones). The residual stream h is updated in place: each RMSNorm
        kernel first adds the previous sublayer's output to it, as the fp32 split partials of its output
        projection. For up to 64 rows the RMSNorm kernels and the gate / up projection (SwiGLU in its
        epilogue) write their outputs in the tiled activation layout that the next projections read, and
        (the fused step) the attention's output projection adds into h itself and writes h tiled, and the
        gate / up launch normalises its rows (the FFN norm's weight folded into its weight): one RMSNorm
        launch per layer instead of two."""
        eps = self.args.norm_eps
        B = tokens.shape[0]
        xt = self._tiled_acts
        h = self.tok_embeddings[tokens]                                  # [B, dim]
        f = None                                                         # fp32 split partials [ks, B, dim]
        if self._fused_step:
            ht = torch.empty(64, self.args.dim, dtype=h.dtype, device=h.device)   # h, tiled
            for L in self.layers:
                y = decoder_ops.rmsnorm(h, L["attn_norm"], eps, res_part=f, h_out=h, tiled_out=True)
                L["attn"].forward_decode(y, current_pos, x_tiled=True, residual=(h, ht))
                a = L["w13"].swiglu_rmsnorm(ht, eps, x_tiled=True, rows=B)  # silu(gate) * up of rmsnorm(h)
                f = L["w2"](a, x_tiled=True, rows=B, mode="partials")
            y = decoder_ops.rmsnorm(h, self.norm_w, eps, res_part=f, tiled_out=True)
            if greedy:
                return self.output.argmax(y, x_tiled=True, rows=B)              # the logits are not written
            return self.output(y, x_tiled=True, rows=B).float()
        for L in self.layers:
            y = decoder_ops.rmsnorm(h, L["attn_norm"], eps, res_part=f, h_out=h, tiled_out=xt)
            o = L["attn"].forward_decode(y, current_pos, x_tiled=xt, out_partials=True)
            y = decoder_ops.rmsnorm(h, L["ffn_norm"], eps, res_part=o, h_out=h, tiled_out=xt)
            a = L["w13"](y, x_tiled=xt, rows=B)                           # silu(gate) * up
            at = L["w13"].tiled                                          # a tiled gate / up writes tiled rows
            if at and not L["w2"].tiled:
                a, at = decoder_ops.untile_rows(a, B), False
            f = L["w2"](a, x_tiled=at, rows=B, mode="partials")
        y = decoder_ops.rmsnorm(h, self.norm_w, eps, res_part=f, tiled_out=xt)
        logits = self.output(y, x_tiled=xt, rows=B)
        return decoder_ops.argmax_rows(logits) if greedy else logits.float()

    @torch.no_grad()
    def decode_graph(self, tokens: torch.Tensor, current_pos: torch.Tensor, greedy: bool = False) -> torch.Tensor:
        """decode() replayed from a HIP graph captured on first use (one graph per value of greedy); tokens
        and current_pos are copied into the graph's static inputs (the caller's tensors may change between
        steps). The returned tensor is the graph's output buffer, rewritten by the next replay."""
        if self._graph is None:
            self._graph = {}
        if greedy not in self._graph:
            if not hasattr(self, "_tok"):
                self._tok = tokens.clone()
                self._pos = current_pos.clone()
            s = torch.cuda.Stream(self.device)
            s.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(s):
                self.decode(self._tok, self._pos, greedy)                # sets kernel attributes outside capture
            torch.cuda.current_stream(self.device).wait_stream(s)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                out = self.decode(self._tok, self._pos, greedy)
            self._graph[greedy] = (g, out)
        g, out = self._graph[greedy]
        self._tok.copy_(tokens)
        self._pos.copy_(current_pos)
        g.replay()
        return out


def draw_ranks(n_layers: int, seed: int, lo: int = 32, hi: int = 128, step: int = 8, mean: float = 64.0) -> List[int]:
    """Per-layer ranks in [lo, hi] in steps of `step`, mean about `mean`: lo + step * Binomial(n, p) with
    n = (hi - lo) / step and p chosen for the mean."""
    g = torch.Generator().manual_seed(seed)
    n = (hi - lo) // step
    p = (mean - lo) / (hi - lo)
    return [lo + step * int(torch.bernoulli(torch.full((n,), p), generator=g).sum()) for _ in range(n_layers)]


def random_palu_state_dict(args: ModelArgs, ranks_k: List[int], ranks_v: List[int], device, seed: int = 0,
                           std: float = 0.02, rank_multiple: int = 32, dense_out: Optional[list] = None,
                           use_fused_k: bool = True, rank_multiple_v: Optional[int] = None) -> dict:
    """Random-init weights N(0, std) generated on `device`, and per-layer per-head SVD factors of the
    k / v projections at the given ranks (on `device` too), zero-padded to a multiple of rank_multiple
    (convert.load_palu_dir's padding; V ranks to a multiple of rank_multiple_v when given: 16 suits tiled
    caches, whose V tiles are 16 wide). Every tensor is left in bf16 on `device`. Sets args.palu, whose
    runtime takes the fused latent decode unless use_fused_k is False. With dense_out, every layer's fp32
    projections (HF head order) and padded factors are appended to it as (W, LowRank) on the host."""
    g = torch.Generator(device=device).manual_seed(seed)
    bf = torch.bfloat16
    randn = lambda *s: torch.randn(*s, device=device, generator=g) * std
    hd, nh, nkv, dim = args.head_dim, args.n_heads, args.n_kv_heads, args.dim
    sd = {"tok_embeddings.weight": randn(args.vocab_size, dim).to(bf), "output.weight": randn(args.vocab_size, dim).to(bf),
          "norm.weight": torch.ones(dim, dtype=bf, device=device)}
    pad = lambda r, m: int(math.ceil(r / m) * m)
    rk_pad, rv_pad = [], []
    for i in range(args.n_layers):
        W = {"q": randn(nh * hd, dim), "k": randn(nkv * hd, dim), "v": randn(nkv * hd, dim), "o": randn(dim, nh * hd)}
        fac = []
        for w, r, m in ((W["k"], ranks_k[i], rank_multiple), (W["v"], ranks_v[i], rank_multiple_v or rank_multiple)):
            U, VT = compress.svd_per_head(w, nkv, r)
            rp = min(pad(r, m), hd)
            fac += [F.pad(VT, (0, 0, 0, rp - r)), F.pad(U, (0, rp - r))]
        lr = convert.LowRank(*fac)
        rk_pad.append(lr.r_k)
        rv_pad.append(lr.r_v)
        p = f"layers.{i}"
        sd[f"{p}.attention.wq.weight"] = convert.reverse_permute(W["q"], nh, nh * hd, dim).to(bf)
        sd[f"{p}.attention.wo.weight"] = W["o"].to(bf)
        for name, t in convert.palu_layer_tensors(W, lr, nh, nkv, hd).items():
            sd[f"{p}.attention.palu.{name}"] = t.to(bf)
        if dense_out is not None:
            dense_out.append(({k: v.cpu() for k, v in W.items()},
                              convert.LowRank(*[t.cpu() for t in (lr.k_VT, lr.k_U, lr.v_VT, lr.v_U)])))
        del W, lr, fac
        sd[f"{p}.attention_norm.weight"] = torch.ones(dim, dtype=bf, device=device)
        sd[f"{p}.ffn_norm.weight"] = torch.ones(dim, dtype=bf, device=device)
        sd[f"{p}.feed_forward.w1.weight"] = randn(args.ffn_dim, dim).to(bf)
        sd[f"{p}.feed_forward.w3.weight"] = randn(args.ffn_dim, dim).to(bf)
        sd[f"{p}.feed_forward.w2.weight"] = randn(dim, args.ffn_dim).to(bf)
    args.palu = convert.PaluConfig(rank_k=rk_pad, rank_v=rv_pad, cache_id=f"random-seed{seed}",
                                   runtime=convert.PaluRuntime(use_fused_k=use_fused_k))
    return sd


@torch.no_grad()
def prefill_all(model: Transformer, prompts: torch.Tensor, users_per_chunk: int = 4) -> torch.Tensor:
    """Prefill every cache row from prompts [B, S], users_per_chunk rows per pass (bounds the prefill
    activations); returns the last-position logits [B, vocab]."""
    outs = [model.prefill(prompts[u:u + users_per_chunk], user_id=u)
            for u in range(0, prompts.shape[0], users_per_chunk)]
    return torch.cat(outs)


@torch.no_grad()
def generate(model: Transformer, prompts: torch.Tensor, n_new: int, use_graph: bool = True,
             deterministic: Optional[bool] = None):
    """Greedy decode (reference generate.py:53-62): prefill every row's prompt, then n_new steps of
    argmax sampling. prompts [B, S] with B == max_batch_size. Returns the generated ids [B, n_new].
    deterministic (PaluRuntime.deterministic when given) fixes the decode kernels' block order so that
    the same prompts give the same ids on every run; by default the order is dynamic and a random-init
    model's near-tied logits can pick different ids from run to run."""
    B, S = prompts.shape
    assert B == model.args.max_batch_size and S + n_new <= model.args.max_seq_len
    if deterministic is not None:
        model.set_deterministic(deterministic)
    tok = prefill_all(model, prompts).argmax(-1)
    out = [tok]
    pos = torch.full((B,), S, dtype=torch.int32, device=model.device)
    step = model.decode_graph if use_graph else model.decode
    for t in range(n_new - 1):
        tok = step(tok, pos, greedy=True).clone()                    # argmax of the step's logits
        out.append(tok)
        pos += 1
    return torch.stack(out, dim=1)
