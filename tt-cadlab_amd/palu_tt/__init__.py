"""Palu fused latent flash-decode on MI355X (gfx950).

The reference's palu_tt API surface (fused op entry, weight layout, attention drop-in) over
hand-written HIP kernels in libpalu_mi355x.so. Import path: add tt-cadlab_amd/ to sys.path.
"""
__all__ = ["fused"]
