"""Build the HIP library libpalu_mi355x.so in-tree (hipcc, gfx950 only).

The library is a plain C-ABI shared object (include/palu_mi355x.h); nothing in it links against torch.
``build_native()`` always recompiles (one hipcc process per translation unit, in parallel, then one
link); ``library_path()`` is where the loader looks for the result.
"""
import os
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent                      # tt-cadlab_amd/
REPO = ROOT.parent
CSRC = ROOT / "csrc"
INCLUDE = REPO / "include"
LIB_DIR = PKG_DIR / "_lib"
LIB_NAME = "libpalu_mi355x.so"
SOURCES = ["palu_capi.hip", "palu_decode_rows.hip", "palu_decode_tiled.hip", "palu_decode_rows_paged.hip",
           "palu_decode_tiled_paged.hip", "palu_decode_tiled_k16.hip", "palu_decode_tiled_paged_k16.hip",
           "palu_decode_full.hip", "palu_glrd.hip", "palu_glrd_narrow.hip", "palu_decoder.hip", "palu_linear.hip"]
HEADERS = ["palu_kernel.h", "palu_glrd_scores.h"]
# Per-file flags: the narrow-rank grouped-latent scores kernels keep their MFMA results in VGPRs.
SOURCE_FLAGS = {"palu_glrd_narrow.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
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


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that line is expected.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln and ln.strip()]
    return res.returncode, msgs


def build_native(verbose: bool = False, extra_flags=(), jobs: int = 0) -> Path:
    """Compile every HIP translation unit and link them into one shared library; returns its path."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    out = library_path()
    tmp = out.with_suffix(".so.tmp")
    jobs = jobs or min(len(SOURCES), max(1, min(16, os.cpu_count() or 1)))
    with tempfile.TemporaryDirectory(prefix="palu_build_") as td:
        objs = [Path(td) / (Path(s).stem + ".o") for s in SOURCES]
        cmds = [[hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(s, []), *extra_flags, f"-I{INCLUDE}", "-c", str(CSRC / s),
                 "-o", str(o)]
                for s, o in zip(SOURCES, objs)]
        if verbose:
            for c in cmds:
                print(" ".join(c), flush=True)
        with ThreadPoolExecutor(max_workers=jobs) as ex:
            results = list(ex.map(_run, cmds))
        errs = [(s, m) for s, (rc, m) in zip(SOURCES, results) if rc != 0]
        if errs:
            raise RuntimeError("hipcc failed:\n" + "\n".join(f"[{s}]\n" + "\n".join(m) for s, m in errs))
        link = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *[str(o) for o in objs], "-o", str(tmp)]
        rc, msgs = _run(link)
        if rc != 0:
            raise RuntimeError("link failed:\n" + "\n".join(msgs))
        if verbose:
            for _, (_, m) in zip(SOURCES, results):
                if m:
                    print("\n".join(m), flush=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build_native(verbose=True))
