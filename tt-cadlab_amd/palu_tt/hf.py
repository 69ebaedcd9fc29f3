"""Minimal reader of a local HF checkpoint directory (config.json + *.safetensors shards).

Mirrors the loading helpers the reference uses (palu_tt/hf.py:22-43): no network, no snapshot
download; ``hf_dir`` is a directory on disk.
"""
import json
from pathlib import Path
from typing import Callable, Dict

import torch
from safetensors import safe_open


def load_config(hf_dir: Path) -> dict:
    return json.loads((Path(hf_dir) / "config.json").read_text())


def load_tensors(hf_dir: Path, keep: Callable[[str], bool]) -> Dict[str, torch.Tensor]:
    """Every tensor whose name satisfies ``keep``, from every *.safetensors file of the directory."""
    out = {}
    for f in sorted(Path(hf_dir).glob("*.safetensors")):
        with safe_open(str(f), framework="pt") as sf:
            for k in sf.keys():
                if keep(k):
                    out[k] = sf.get_tensor(k)
    return out
