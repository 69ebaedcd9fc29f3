"""Decode-path fidelity of the fused latent kernel: the same model decoded through the naive path and
through the fused op, teacher-forced, logits compared per step (the reference's harness,
palu_tt/decode_check.py:47-133).

Both paths share one prefill (the fused op replaces decode only, so the prefill logits are identical and
are left out of the comparison, as the reference leaves them out). Then every row is fed the same
teacher tokens one decode step at a time, first through the naive path (K rebuilt for recon_len positions
and rotated, stock flash-decode) and then through the fused op. Decode step t writes cache position
prompt_len + t before it reads positions <= prompt_len + t, so a later pass overwrites what an earlier one
wrote and reads nothing stale. Reported per step: the minimum over rows of the logit PCC, and how often
the argmax agrees.

A caller may add a third pass through its own attention core (``reference_core(layer, q4, keys, values,
pos) -> [1, B, nh, out_width]``; ``fp32_attention_core`` below is plain fp32 attention over the same
latent caches): both paths are then also compared with it, which separates a path's own error from the
run-to-run spread of the model.
"""
import argparse
import json
import types
from pathlib import Path
from typing import Callable, Dict, Optional

import torch

from palu_tt import fused
from palu_tt import model as pm


def fp32_attention_core(layer, q4, keys, values, pos):
    """A reference attention core for fused_vs_naive: plain fp32 torch attention over a PaluAttention
    layer's own caches (K = latent @ u_k for the first recon_len positions, Meta RoPE, masked softmax, V
    rebuilt with u_v for grouped latents or attended in latent space), rounded to bf16 like the cores it
    stands beside. [1, B, nh, out_width]."""
    S = layer._recon_len()
    gs, nkv, nh, hd = layer.gs, layer.n_kv_heads, layer.n_heads, layer.head_dim
    per_head = (lambda t: t) if gs == 1 else (lambda t: t.repeat_interleave(gs, dim=1))
    if layer.recon_k:
        K = per_head(layer._cache_rows(keys, S)).float() @ layer.u_k.float()                 # [B, nkv, S, hd]
        K = fused.apply_rope_meta(K, layer.cos[:S][None, None], layer.sin[:S][None, None])
    else:
        K = layer._cache_rows(keys, S).float()                                                # rotated full K
    V = layer._cache_rows(values, S).float()
    if gs > 1:
        V = per_head(V) @ layer.u_v.float()
    B = q4.shape[1]
    q = q4[0].float().view(B, nkv, nh // nkv, hd)
    sc = (q @ K.transpose(-1, -2)) * layer.scale                                               # [B, nkv, rep, S]
    masked = torch.arange(S, device=q.device)[None, :] > pos.long()[:, None]
    sc = sc.masked_fill(masked[:, None, None, :], float("-inf"))
    return (torch.softmax(sc, dim=-1) @ V).reshape(1, B, nh, -1).to(torch.bfloat16)


def _pcc_rows(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Pearson correlation of each row of a with the same row of b ([rows, n] -> [rows]), in fp64."""
    a = a.double() - a.double().mean(-1, keepdim=True)
    b = b.double() - b.double().mean(-1, keepdim=True)
    return (a * b).sum(-1) / (a.norm(dim=-1) * b.norm(dim=-1)).clamp_min(1e-300)


def _compare(x: torch.Tensor, y: torch.Tensor) -> Dict[str, object]:
    pcc = torch.stack([_pcc_rows(x[t], y[t]) for t in range(x.shape[0])])     # [T, B]
    return {"pcc_min_per_step": [round(float(v), 6) for v in pcc.min(dim=1).values],
            "pcc_min": float(pcc.min()), "pcc_mean": float(pcc.mean()),
            "argmax_agree": float((x.argmax(-1) == y.argmax(-1)).double().mean())}


@torch.no_grad()
def fused_vs_naive(model: "pm.Transformer", prompts: torch.Tensor, teacher: torch.Tensor, use_graph: bool = False,
                   reference_core: Optional[Callable] = None) -> Dict[str, object]:
    """prompts [B, P] and teacher [B, T] token ids on the model's device (B == max_batch_size). Returns
    {"steps": T, "rows": B, "pcc_min_per_step": [...], "pcc_min", "pcc_mean", "argmax_agree"} for fused vs
    naive, and with reference_core also "fused_vs_reference" and "naive_vs_reference" in the same form."""
    B, P = prompts.shape
    T = teacher.shape[1]
    assert B == model.args.max_batch_size and P + T <= model.args.max_seq_len
    pm.prefill_all(model, prompts)

    def decode_pass(use_fused_k: bool, graph: bool) -> torch.Tensor:
        model.set_fused_k(use_fused_k, recon_len=P + T)
        step = model.decode_graph if graph else model.decode
        pos = torch.full((B,), P, dtype=torch.int32, device=model.device)
        logits = []
        for t in range(T):
            logits.append(step(teacher[:, t], pos).clone())
            pos += 1
        return torch.stack(logits)                                       # [T, B, vocab] fp32

    naive = decode_pass(False, use_graph)
    fused_l = decode_pass(True, use_graph)
    out = {"steps": T, "rows": B, **_compare(naive, fused_l)}
    if reference_core is not None:
        layers = [L["attn"] for L in model.layers]
        for att in layers:   # the reference core answers row-major whatever layout the layer asks for
            att.decode_core = types.MethodType(
                lambda self, q4, keys, values, pos, tiled_rows=False: reference_core(self, q4, keys, values, pos), att)
        try:
            ref = decode_pass(False, False)
        finally:
            for att in layers:
                del att.decode_core                                      # back to the class's method
        out["fused_vs_reference"] = _compare(fused_l, ref)
        out["naive_vs_reference"] = _compare(naive, ref)
    model.set_fused_k(True)
    return out


def main(argv=None) -> Dict[str, object]:
    """Command line: ``python -m palu_tt.decode_check --row NAME [--steps 64] [--out DIR]``, the
    reference's harness (palu_tt/decode_check.py:62-134) on a Llama-3.1-8B-shaped Palu model. There are
    no checkpoints or datasets here, so the weights are seeded random-init with per-layer SVD factors
    (ranks drawn as the benchmark draws them) and the prompt and teacher tokens are seeded random ids.
    --steps counts the decode steps compared (the reference's counts the prefill step too and reports
    one less). Prints one JSON line; with --out also writes it to DIR/decode_check_<row>.json."""
    p = argparse.ArgumentParser(description=main.__doc__.splitlines()[0])
    p.add_argument("--row", required=True, help="name of the result row")
    p.add_argument("--steps", type=int, default=63, help="teacher-forced decode steps compared")
    p.add_argument("--batch", type=int, default=1)
    p.add_argument("--prompt", type=int, default=512, help="prompt tokens prefilled before the decode steps")
    p.add_argument("--layers", type=int, default=32)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--graph", action="store_true", help="decode steps as HIP graphs")
    p.add_argument("--fp32-core", action="store_true",
                   help="also compare both paths with plain fp32 attention over the same caches")
    p.add_argument("--out", default=None, help="directory for decode_check_<row>.json")
    a = p.parse_args(argv)
    dev = torch.device("cuda:0")
    L, B, P, T = a.layers, a.batch, a.prompt, a.steps
    args = pm.ModelArgs(n_layers=L, max_batch_size=B, max_seq_len=(P + T + 32) // 32 * 32)
    ranks_k, ranks_v = pm.draw_ranks(L, seed=1), pm.draw_ranks(L, seed=2)
    sd = pm.random_palu_state_dict(args, ranks_k, ranks_v, dev, seed=a.seed, rank_multiple=16)
    model = pm.Transformer(args, sd, dev)
    del sd
    g = torch.Generator().manual_seed(a.seed + 7)
    prompts = torch.randint(0, args.vocab_size, (B, P), generator=g).to(dev)
    teacher = torch.randint(0, args.vocab_size, (B, T), generator=g).to(dev)
    r = fused_vs_naive(model, prompts, teacher, use_graph=a.graph,
                       reference_core=fp32_attention_core if a.fp32_core else None)
    out = {"row": a.row, "weights": "random-init, seeded", "layers": L, "batch": B, "prompt": P,
           "ranks_k": ranks_k, "ranks_v": ranks_v, "graph": bool(a.graph), **r}
    line = json.dumps(out)
    print(line, flush=True)
    if a.out:
        d = Path(a.out)
        d.mkdir(parents=True, exist_ok=True)
        (d / f"decode_check_{a.row}.json").write_text(json.dumps(out, indent=1))
    return out


if __name__ == "__main__":
    main()
