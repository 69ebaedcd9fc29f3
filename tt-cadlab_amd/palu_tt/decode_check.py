"""Decode-path fidelity of the fused latent kernel: the same model decoded through the naive path and
through the fused op, teacher-forced, logits compared per step (the reference's harness,
palu_tt/decode_check.py:47-133).

Both paths share one prefill (the fused op replaces decode only, so the prefill logits are identical and
are left out of the comparison, as the reference leaves them out). Then every row is fed the same
teacher tokens one decode step at a time, first through the naive path (K rebuilt for recon_len positions
and rotated, stock flash-decode) and then through the fused op. Decode step t writes cache position
prompt_len + t before it reads positions <= prompt_len + t, so the second pass overwrites what the first
wrote and reads nothing stale. Reported per step: the minimum over rows of the logit PCC, and how often
the argmax agrees.
"""
from typing import Dict

import torch

from palu_tt import model as pm


def _pcc_rows(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Pearson correlation of each row of a with the same row of b ([rows, n] -> [rows]), in fp64."""
    a = a.double() - a.double().mean(-1, keepdim=True)
    b = b.double() - b.double().mean(-1, keepdim=True)
    return (a * b).sum(-1) / (a.norm(dim=-1) * b.norm(dim=-1)).clamp_min(1e-300)


@torch.no_grad()
def fused_vs_naive(model: "pm.Transformer", prompts: torch.Tensor, teacher: torch.Tensor,
                   use_graph: bool = False) -> Dict[str, object]:
    """prompts [B, P] and teacher [B, T] token ids on the model's device (B == max_batch_size). Returns
    {"steps": T, "pcc_min_per_step": [...], "pcc_min": x, "pcc_mean": x, "argmax_agree": x}."""
    B, P = prompts.shape
    T = teacher.shape[1]
    assert B == model.args.max_batch_size and P + T <= model.args.max_seq_len
    pm.prefill_all(model, prompts)
    runs = {}
    for fused in (False, True):
        model.set_fused_k(fused, recon_len=P + T)
        step = model.decode_graph if use_graph else model.decode
        pos = torch.full((B,), P, dtype=torch.int32, device=model.device)
        logits = []
        for t in range(T):
            logits.append(step(teacher[:, t], pos).clone())
            pos += 1
        runs[fused] = torch.stack(logits)                        # [T, B, vocab] fp32
    model.set_fused_k(True)
    naive, fused_l = runs[False], runs[True]
    pcc = torch.stack([_pcc_rows(naive[t], fused_l[t]) for t in range(T)])   # [T, B]
    agree = (naive.argmax(-1) == fused_l.argmax(-1)).double().mean()
    return {"steps": T, "rows": B, "pcc_min_per_step": [round(float(x), 6) for x in pcc.min(dim=1).values],
            "pcc_min": float(pcc.min()), "pcc_mean": float(pcc.mean()), "argmax_agree": float(agree)}
