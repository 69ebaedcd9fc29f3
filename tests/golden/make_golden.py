#!/usr/bin/env python
"""Writes tests/golden/decode_small.safetensors: inputs and the oracle's fp32 output of one fused
latent decode on a small ragged batch.

The output comes from oracle.palu_oracle.reference_decode, which tests/test_oracle.py pins against
transformers' rotary embedding and attention, brute-force loops and the reference's own test
properties. The fixture freezes those pinned values so the oracle cannot drift silently, and gives the
GPU path an input/output pair it must reproduce. Run from the repository root:

    python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO))
from oracle import palu_oracle as ref  # noqa: E402

HD = 128
THETA = 500000.0
LLAMA3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}
B, NQ, NKV, S, RK, RV = 3, 8, 2, 128, 64, 32
CUR_POS = [37, 95, 127]          # ragged rows: a partial block, a mid-cache end, the full cache


def make():
    g = torch.Generator().manual_seed(213919)
    bf = lambda *s, std=1.0: (torch.randn(*s, generator=g) * std).to(torch.bfloat16)
    q = bf(1, B, NQ, HD, std=1.3)
    k_lat = bf(B, NKV, S, RK)
    v_lat = bf(B, NKV, S, RV)
    u_k = bf(NKV, RK, HD, std=0.15)
    cur = torch.tensor(CUR_POS, dtype=torch.int32)
    cos, sin = ref.cos_sin_tables(HD, S, THETA, LLAMA3)
    out = ref.reference_decode(q.float(), k_lat.float(), u_k.float(), v_lat.float(), cur, cos, sin, HD ** -0.5)
    return {"q": q, "k_latent": k_lat, "v_latent": v_lat, "u_k": u_k, "cur_pos": cur, "out": out.float().contiguous()}


if __name__ == "__main__":
    path = Path(__file__).resolve().parent / "decode_small.safetensors"
    save_file(make(), str(path), metadata={"theta": str(THETA), "rope": "llama3 factor 8, low 1, high 4, orig 8192",
                                           "scale": "head_dim ** -0.5", "generator": "tests/golden/make_golden.py"})
    print(f"wrote {path} ({path.stat().st_size} bytes)")
