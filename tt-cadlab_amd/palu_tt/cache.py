"""Latent KV caches in the MI355X tiled HBM layout.

The reference keeps each latent cache as a [B, n_groups, max_seq, r] device tensor
(palu_tt/attention.py:274-283) and appends one row per decode step with paged_update_cache
(attention.py:622-623). ``LatentCache`` holds the same logical tensor in the layout the fused decode
streams fastest: every 32-position block is (2 * r / 32) tiles of 1 KB, each tile already in the
operand order of the kernel's MFMAs, so a wave reads one contiguous KB per load instruction.

Tile (c, kb) of block blk, slot l = 16*g + n (g < 4, n < 16), holds the 8 values r-index 32*kb + 8*g
.. +7 of position 32*blk + 8*(n//4) + 4*c + n%4. The storage tensor is [B, G, S/32, 2*r/32, 64, 8]
bf16; ``from_rows`` / ``to_rows`` convert to and from the logical row-major tensor.
"""
from dataclasses import dataclass
from typing import Tuple

import torch

BLOCK = 32


def rows_to_tiled(rows: torch.Tensor) -> torch.Tensor:
    """[B, G, S, r] -> tiled storage [B, G, S/32, 2*r/32, 64, 8] (same dtype, new contiguous tensor)."""
    B, G, S, r = rows.shape
    assert S % BLOCK == 0 and r % 32 == 0, f"tiled layout needs S % 32 == 0 and r % 32 == 0, got S={S}, r={r}"
    # position 32*blk + 8*tb + 4*c + i, r-index 32*kb + 8*g + j  ->  [blk][c][kb][g][tb][i][j]
    x = rows.reshape(B, G, S // BLOCK, 4, 2, 4, r // 32, 4, 8)
    x = x.permute(0, 1, 2, 4, 6, 7, 3, 5, 8)
    return x.reshape(B, G, S // BLOCK, 2 * r // 32, 64, 8).contiguous()


def tiled_to_rows(tiled: torch.Tensor) -> torch.Tensor:
    """Inverse of rows_to_tiled."""
    B, G, nblk, ntile, _, _ = tiled.shape
    r = ntile * 16
    x = tiled.reshape(B, G, nblk, 2, r // 32, 4, 4, 4, 8)          # [blk][c][kb][g][tb][i][j]
    x = x.permute(0, 1, 2, 6, 3, 7, 4, 5, 8)                      # [blk][tb][c][i][kb][g][j]
    return x.reshape(B, G, nblk * BLOCK, r).contiguous()


@dataclass
class LatentCache:
    """A latent cache of logical shape [B, n_groups, max_seq, width] in the tiled layout."""
    data: torch.Tensor

    @staticmethod
    def zeros(batch: int, n_groups: int, max_seq: int, width: int, device, dtype=torch.bfloat16) -> "LatentCache":
        assert max_seq % BLOCK == 0, f"max_seq must be a multiple of {BLOCK}, got {max_seq}"
        assert width % 32 == 0, f"width must be a multiple of 32, got {width}"
        return LatentCache(torch.zeros(batch, n_groups, max_seq // BLOCK, 2 * width // 32, 64, 8, dtype=dtype,
                                       device=device))

    @staticmethod
    def from_rows(rows: torch.Tensor) -> "LatentCache":
        return LatentCache(rows_to_tiled(rows))

    def to_rows(self) -> torch.Tensor:
        return tiled_to_rows(self.data)

    @property
    def shape(self) -> Tuple[int, int, int, int]:
        B, G, nblk, ntile = self.data.shape[:4]
        return (B, G, nblk * BLOCK, ntile * 16)

    @property
    def device(self):
        return self.data.device

    @property
    def dtype(self):
        return self.data.dtype

    def data_ptr(self) -> int:
        return self.data.data_ptr()

    def nbytes(self) -> int:
        return self.data.numel() * self.data.element_size()
