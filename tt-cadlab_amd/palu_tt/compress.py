"""Truncated SVD of k_proj / v_proj into Palu factors, per head (M-LRD) or per head group (G-LRD).

``svd_per_head`` keeps the reference's factor convention (palu_tt/compress.py:12-23): Palu's balanced
split U = U_r sqrt(S), VT = sqrt(S) Vt_r. ``svd_per_group`` factors the stacked rows of each group of
heads jointly, which is the G-LRD form (one latent per group, one U slice per head), and
``factor_layers`` turns per-layer projection weights into the per-group factor lists that
``palu_tt.convert.save_palu_dir`` writes in the on-disk format ``load_palu_dir`` reads.
"""
from typing import Dict, List, Sequence, Tuple

import torch


def svd_per_group(W: torch.Tensor, n_groups: int, rank: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """W [n_groups * rows, dim] -> U [n_groups, rows, rank], VT [n_groups, rank, dim], with each group's
    rows W_g ~= U_g @ VT_g (exact when rank >= min(rows, dim)); one batched SVD over the groups."""
    rows = W.shape[0] // n_groups
    U, S, Vt = torch.linalg.svd(W.float().reshape(n_groups, rows, -1), full_matrices=False)
    root = S[:, :rank].sqrt()
    return U[:, :, :rank] * root[:, None, :], root[:, :, None] * Vt[:, :rank, :]


def svd_per_head(W: torch.Tensor, n_heads: int, rank: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """W [n_heads*hd, dim] -> U [n_heads, hd, rank], VT [n_heads, rank, dim] with W_h ~= U_h @ VT_h."""
    return svd_per_group(W, n_heads, rank)


def factor_layers(weights: Dict[int, Dict[str, torch.Tensor]], n_kv_heads: int, ranks_k: Sequence[Sequence[int]],
                  ranks_v: Sequence[Sequence[int]]) -> Dict[int, Dict[str, List[Tuple[torch.Tensor, torch.Tensor]]]]:
    """weights[i] = {"k": W_k, "v": W_v} ([n_kv * hd, hidden] each, HF head order); ranks_k[i] / ranks_v[i]
    list one rank per head group (len = n_groups; group size n_kv / n_groups). Returns layers[i][proj] =
    [(U_g, VT_g)] per group, the input of convert.save_palu_dir."""
    out = {}
    for i, w in weights.items():
        out[i] = {}
        for proj, W, group_ranks in (("k_proj", w["k"], ranks_k[i]), ("v_proj", w["v"], ranks_v[i])):
            n_groups = len(group_ranks)
            if n_kv_heads % n_groups:
                raise ValueError(f"layer {i} {proj}: {n_groups} groups do not divide {n_kv_heads} KV heads")
            U, VT = svd_per_group(W, n_groups, max(group_ranks))
            out[i][proj] = [(U[g, :, :r].contiguous(), VT[g, :r].contiguous()) for g, r in enumerate(group_ranks)]
    return out
