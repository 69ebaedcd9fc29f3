"""The committed fixture tests/golden/decode_small.safetensors (written by tests/golden/make_golden.py):
the oracle must still produce it (CPU), and the HIP op must reproduce it from the stored inputs (GPU),
in both cache layouts, to the decode bar (max-abs 2e-2, cosine 0.9999)."""
from pathlib import Path

import pytest
import torch
from safetensors.torch import load_file

from oracle import palu_oracle as ref

GOLDEN = Path(__file__).resolve().parent / "golden" / "decode_small.safetensors"
HD = 128
THETA = 500000.0
LLAMA3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}


@pytest.fixture(scope="module")
def fx():
    return load_file(str(GOLDEN))


def test_oracle_reproduces_the_fixture(fx):
    S = fx["k_latent"].shape[2]
    cos, sin = ref.cos_sin_tables(HD, S, THETA, LLAMA3)
    out = ref.reference_decode(fx["q"].float(), fx["k_latent"].float(), fx["u_k"].float(), fx["v_latent"].float(),
                               fx["cur_pos"], cos, sin, HD ** -0.5)
    torch.testing.assert_close(out, fx["out"], atol=2e-6, rtol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["rows", "tiled"])
def test_hip_op_reproduces_the_fixture(gpu, fx, layout):
    from palu_tt import fused
    from palu_tt.cache import LatentCache
    S = fx["k_latent"].shape[2]
    cos, sin = fused.cos_sin_tables(HD, S, THETA, LLAMA3)
    k, v = fx["k_latent"].to(gpu), fx["v_latent"].to(gpu)
    if layout == "tiled":
        k, v = LatentCache.from_rows(k, "k"), LatentCache.from_rows(v, "v")
    out = fused.palu_sdpa_decode(fx["q"].to(gpu), k, fused.w_rot_from_u_k(fx["u_k"].float()).to(gpu, torch.bfloat16)[None],
                                 fused.cs_table(cos, sin, S)[None, None].to(gpu), v, fx["v_latent"].shape[-1],
                                 fx["cur_pos"].to(gpu), scale=HD ** -0.5, out_dtype=torch.float32, deterministic=True)
    torch.cuda.synchronize()
    out = out.cpu()
    assert ref.max_abs(out, fx["out"]) <= 2e-2 and ref.cosine(out, fx["out"]) >= 0.9999, \
        (ref.max_abs(out, fx["out"]), ref.cosine(out, fx["out"]))
