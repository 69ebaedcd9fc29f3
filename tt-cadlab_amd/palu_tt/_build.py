"""Build the HIP library libpalu_mi355x.so in-tree (hipcc, gfx950 only).

The library is a plain C-ABI shared object (include/palu_mi355x.h); nothing in it links against torch.
``build_native()`` always recompiles; ``library_path()`` is where the loader looks for the result.
"""
import os
import shutil
import subprocess
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent                      # tt-cadlab_amd/
REPO = ROOT.parent
CSRC = ROOT / "csrc"
INCLUDE = REPO / "include"
LIB_DIR = PKG_DIR / "_lib"
LIB_NAME = "libpalu_mi355x.so"
SOURCES = ["palu_decode.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Packed fp32 VALU ops stay off in all device code (the compiler would otherwise form
    # v_pk_{add,mul,fma}_f32 from float pairs).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def library_path() -> Path:
    return LIB_DIR / LIB_NAME


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the MI355X library needs ROCm's hipcc to build")


def build_native(verbose: bool = False, extra_flags=()) -> Path:
    """Compile every HIP source into one shared library; returns its path."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    out = library_path()
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, *extra_flags, f"-I{INCLUDE}", *[str(CSRC / s) for s in SOURCES], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that line is expected.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln and ln.strip()]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs), flush=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build_native(verbose=True))
