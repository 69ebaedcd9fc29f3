"""ctypes binding of libpalu_mi355x.so (declarations: include/palu_mi355x.h).

The library is found in palu_tt/_lib/ (built in-tree by palu_tt._build.build_native). There is no
fallback: when the library is missing or a call fails, a RuntimeError carries the library's message.
torch is imported first so that the library binds to the HIP runtime torch already loaded (both are
libamdhip64.so.7), which keeps torch's streams and device pointers valid across the boundary.
"""
import ctypes
import threading

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

from palu_tt._build import library_path

PALU_OK, PALU_EINVAL, PALU_EUNSUPPORTED, PALU_EHIP = 0, 1, 2, 3
DTYPE_F32, DTYPE_BF16 = 0, 1
OUT_TILED_ROWS = 0x100      # PALU_OUT_TILED_ROWS, OR'ed into palu_sdpa_decode's out_dtype
ABI_VERSION = 14
LAYOUT_ROWS, LAYOUT_TILED, LAYOUT_TILED_V, LAYOUT_TILED_GROUPED = 0, 1, 2, 3

_vp, _i, _f, _sz, _ll = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_longlong

_SIGNATURES = {
    "palu_last_error": (ctypes.c_char_p, []),
    "palu_abi_version": (_i, []),
    "palu_decode_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "palu_glrd_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "palu_sdpa_decode": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _f, _i, _i, _i, _i,
                              _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "palu_sdpa_decode_noalloc": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _f, _i, _i, _i,
                                      _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "palu_flash_decode": (_i, [_vp, _vp, _vp, _vp, _vp, _f, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "palu_latent_append": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "palu_sdpa_decode_paged": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _f, _i, _i, _i, _i,
                                    _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "palu_flash_decode_paged": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _f, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i,
                                     _vp, _sz, _vp]),
    "palu_latent_append_paged": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "palu_latent_append_strided": (_i, [_vp, _vp, _ll, _ll, _vp, _i, _i, _i, _i, _i, _vp]),
    "palu_latent_append_grouped": (_i, [_vp, _vp, _ll, _ll, _vp, _i, _i, _i, _vp, _i, _vp]),
    "palu_rmsnorm": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _i, _f, _i, _vp]),
    "palu_swiglu": (_i, [_vp, _vp, _i, _i, _i, _vp]),
    "palu_argmax_rows": (_i, [_vp, _ll, _i, _i, _vp, _vp]),
    "palu_rope_rows": (_i, [_vp, _ll, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "palu_linear_tiled": (_i, [_vp, _ll, _i, _i, _vp, _i, _i, _vp, _ll, _i, _i, _i, _vp, _sz, _vp]),
    "palu_qkv_post": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _i, _i, _vp, _vp, _i, _i, _i, _i, _i, _vp, _i, _i, _i, _i,
                           _i, _i, _vp]),
    "palu_linear_plan": (_i, [_i, _i, _i, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]),
    "palu_linear_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "palu_linear_argmax": (_i, [_vp, _ll, _i, _i, _vp, _i, _i, _i, _vp, _vp, _sz, _vp]),
    "palu_linear_argmax_workspace_bytes": (_sz, [_i, _i]),
    "palu_linear_plan_ks": (_i, [_i, _i, _i, _i, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]),
    "palu_linear_swiglu_rmsnorm": (_i, [_vp, _ll, _i, _i, _vp, _i, _i, _i, _f, _vp, _vp]),
    "palu_linear_residual": (_i, [_vp, _ll, _i, _i, _vp, _i, _i, _i, _vp, _ll, _vp, _vp]),
    "palu_linear_qkv": (_i, [_vp, _ll, _i, _i, _vp, _i, _i, _i, _vp, _vp, _vp, _i, _i, _vp, _vp, _i, _i, _i, _i, _i,
                             _vp, _i, _i, _i, _i, _i, _i, _vp]),
}
EXPORTED = tuple(_SIGNATURES)

NOALLOC_SCRATCH_BYTES = 64 << 20     # PALU_NOALLOC_SCRATCH_BYTES

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """The loaded library (loaded once). Raises RuntimeError when it has not been built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            raise RuntimeError(f"{path} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
                               "(or palu_tt._build.build_native()) first")
        lib = ctypes.CDLL(str(path))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        if lib.palu_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{path}: ABI version {lib.palu_abi_version()} != {ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


def check(status: int) -> None:
    if status != PALU_OK:
        msg = load().palu_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"palu library call failed with status {status}")


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def stream_handle(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
