"""Latent KV caches in the MI355X tiled HBM layout.

The reference keeps each latent cache as a [B, n_groups, max_seq, r] device tensor
(palu_tt/attention.py:274-283) and appends one row per decode step with paged_update_cache
(attention.py:622-623). ``LatentCache`` holds the same logical tensor in the layout the fused decode
streams fastest: every 32-position block is r / 16 tiles of 1 KB, each tile already in the operand
order of the kernel's MFMAs, so a wave reads one contiguous KB per load instruction and feeds it to
the matrix cores without any regrouping. The order depends on the cache's role:

  K caches ("k"): tile c * (r/32) + kb, slot l = 16*g + n (g < 4, n < 16) holds r-index 32*kb + 8*g
    .. +7 of block position 8*(n//4) + 4*c + n%4 (the operand of the K rebuild). When r is an odd
    multiple of 16, each half-block c (its 16 * r elements start at c * 16 * r) ends in a 512-byte half
    tile: slot l = 16*g + n holds the 4 r-indices 32*(r//32) + 4*g .. +3 (the low half of the lane's
    operand, zeros above);
  V caches ("v"): tile mt, slot l = 16*g + m holds block positions 8*g .. 8*g + 7 of r-index 16*mt + m
    (the operand of the probability-times-V product).

The storage tensor is [B, G, S/32, r/16, 64, 8] bf16 (one 32-position block is 32 * r elements in that
order); ``from_rows`` / ``to_rows`` convert to and from the logical row-major tensor.
"""
from dataclasses import dataclass
from typing import Tuple

import torch

BLOCK = 32


ROLES = ("k", "v")


def rows_to_tiled(rows: torch.Tensor, role: str = "k") -> torch.Tensor:
    """[B, G, S, r] -> tiled storage [B, G, S/32, r/16, 64, 8] in the role's tile order."""
    B, G, S, r = rows.shape
    assert role in ROLES, f"role must be 'k' or 'v', got {role!r}"
    assert S % BLOCK == 0 and r % 16 == 0, f"tiled {role} layout needs S % 32 == 0 and r % 16 == 0, got S={S}, r={r}"
    nb, kbf = S // BLOCK, r // 32
    if role == "k":
        # position 32*blk + 8*tb + 4*c + i, r-index 32*kb + 8*g + j  ->  [blk][c][kb][g][tb][i][j]
        blk = rows.reshape(B, G, nb, 4, 2, 4, r)
        x = blk[..., :32 * kbf].reshape(B, G, nb, 4, 2, 4, kbf, 4, 8).permute(0, 1, 2, 4, 6, 7, 3, 5, 8)
        x = x.reshape(B, G, nb, 2, kbf * 512)
        if r % 32:
            # half tile: r-index 32*kbf + 4*g + j  ->  [blk][c][g][tb][i][j]
            h = blk[..., 32 * kbf:].reshape(B, G, nb, 4, 2, 4, 4, 4).permute(0, 1, 2, 4, 6, 3, 5, 7)
            x = torch.cat([x, h.reshape(B, G, nb, 2, 256)], dim=-1)
    else:
        # position 32*blk + 8*g + j, r-index 16*mt + m  ->  [blk][mt][g][m][j]
        x = rows.reshape(B, G, nb, 4, 8, r // 16, 16).permute(0, 1, 2, 5, 3, 6, 4)
    return x.reshape(B, G, nb, r // 16, 64, 8).contiguous()


def tiled_to_rows(tiled: torch.Tensor, role: str = "k") -> torch.Tensor:
    """Inverse of rows_to_tiled."""
    B, G, nblk, ntile, _, _ = tiled.shape
    r = ntile * 16
    kbf = r // 32
    if role == "k":
        flat = tiled.reshape(B, G, nblk, 2, 16 * r)               # the two half-blocks c
        x = flat[..., :kbf * 512].reshape(B, G, nblk, 2, kbf, 4, 4, 4, 8)   # [blk][c][kb][g][tb][i][j]
        x = x.permute(0, 1, 2, 6, 3, 7, 4, 5, 8).reshape(B, G, nblk, 4, 2, 4, 32 * kbf)  # [blk][tb][c][i][kb g j]
        if r % 32:
            h = flat[..., kbf * 512:].reshape(B, G, nblk, 2, 4, 4, 4, 4)     # [blk][c][g][tb][i][j]
            h = h.permute(0, 1, 2, 5, 3, 6, 4, 7).reshape(B, G, nblk, 4, 2, 4, 16)  # [blk][tb][c][i][g j]
            x = torch.cat([x, h], dim=-1)
    else:
        x = tiled.reshape(B, G, nblk, r // 16, 4, 16, 8)         # [blk][mt][g][m][j]
        x = x.permute(0, 1, 2, 4, 6, 3, 5)                       # [blk][g][j][mt][m]
    return x.reshape(B, G, nblk * BLOCK, r).contiguous()


@dataclass
class LatentCache:
    """A K ("k") or V ("v") cache of logical shape [B, n_groups, max_seq, width] in the tiled layout."""
    data: torch.Tensor
    role: str = "k"

    def __post_init__(self):
        assert self.role in ROLES, f"role must be 'k' or 'v', got {self.role!r}"

    @staticmethod
    def zeros(batch: int, n_groups: int, max_seq: int, width: int, device, role: str = "k",
              dtype=torch.bfloat16) -> "LatentCache":
        assert max_seq % BLOCK == 0, f"max_seq must be a multiple of {BLOCK}, got {max_seq}"
        assert width % 16 == 0, f"a tiled {role} cache's width must be a multiple of 16, got {width}"
        return LatentCache(torch.zeros(batch, n_groups, max_seq // BLOCK, width // 16, 64, 8, dtype=dtype,
                                       device=device), role)

    @staticmethod
    def from_rows(rows: torch.Tensor, role: str = "k") -> "LatentCache":
        return LatentCache(rows_to_tiled(rows, role), role)

    def to_rows(self) -> torch.Tensor:
        return tiled_to_rows(self.data, self.role)

    def write_rows(self, b: int, start: int, rows: torch.Tensor) -> None:
        """cache[b, :, start:start + n, :] = rows ([G, n, width]); converts only the blocks it touches."""
        G, n, w = rows.shape
        b0, b1 = start // BLOCK, (start + n + BLOCK - 1) // BLOCK
        cur = tiled_to_rows(self.data[b:b + 1, :, b0:b1], self.role)          # [1, G, (b1 - b0) * 32, w]
        cur[0, :, start - b0 * BLOCK:start - b0 * BLOCK + n] = rows.to(cur.dtype)
        self.data[b:b + 1, :, b0:b1] = rows_to_tiled(cur, self.role)

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


@dataclass
class GroupedLatentCache:
    """Grouped latents (G-LRD) whose groups have unequal ranks, stored compactly: group g of every row at
    its own width ranks[g], in the role's tile order, instead of padded to the layer's widest group as
    the reference keeps them (palu_tt/convert.py:178). Row b's group streams lie one after another: the
    storage is [B, S * sum(ranks)] bf16 and group g starts at S * (ranks[0] + .. + ranks[g-1]). The
    logical tensor is the padded [B, n_groups, max_seq, max(ranks)] one, its columns past a group's rank
    zero (``to_rows``); ``from_rows`` keeps each group's first ranks[g] columns."""
    data: torch.Tensor
    ranks: Tuple[int, ...]
    max_seq: int
    role: str = "k"

    def __post_init__(self):
        assert self.role in ROLES, f"role must be 'k' or 'v', got {self.role!r}"
        self.ranks = tuple(int(r) for r in self.ranks)
        assert self.max_seq % BLOCK == 0 and all(r > 0 and r % 16 == 0 for r in self.ranks), \
            f"max_seq a multiple of {BLOCK} and ranks multiples of 16, got {self.max_seq}, {self.ranks}"
        assert self.data.dim() == 2 and self.data.shape[1] == self.max_seq * sum(self.ranks)

    @staticmethod
    def zeros(batch: int, ranks, max_seq: int, device, role: str = "k", dtype=torch.bfloat16) -> "GroupedLatentCache":
        return GroupedLatentCache(torch.zeros(batch, max_seq * sum(int(r) for r in ranks), dtype=dtype, device=device),
                                  tuple(ranks), max_seq, role)

    def _offset(self, g: int) -> int:
        return self.max_seq * sum(self.ranks[:g])

    def group(self, g: int) -> torch.Tensor:
        """Group g's tiled storage as a [B, 1, S/32, ranks[g]/16, 64, 8] view (rows are not contiguous)."""
        B, S, r = self.data.shape[0], self.max_seq, self.ranks[g]
        return self.data[:, self._offset(g):self._offset(g) + S * r].view(B, 1, S // BLOCK, r // 16, 64, 8)

    @staticmethod
    def from_rows(rows: torch.Tensor, ranks, role: str = "k") -> "GroupedLatentCache":
        B, G, S, w = rows.shape
        assert len(ranks) == G and max(ranks) <= w, f"{G} groups of ranks <= {w}, got {ranks}"
        c = GroupedLatentCache.zeros(B, ranks, S, rows.device, role, rows.dtype)
        for g, r in enumerate(c.ranks):
            c.group(g).copy_(rows_to_tiled(rows[:, g:g + 1, :, :r].contiguous(), role))
        return c

    def to_rows(self) -> torch.Tensor:
        B, S, w = self.data.shape[0], self.max_seq, max(self.ranks)
        out = torch.zeros(B, len(self.ranks), S, w, dtype=self.data.dtype, device=self.data.device)
        for g, r in enumerate(self.ranks):
            out[:, g, :, :r] = tiled_to_rows(self.group(g).contiguous(), self.role)[:, 0]
        return out

    def write_rows(self, b: int, start: int, rows: torch.Tensor) -> None:
        """cache[b, :, start:start + n, :] = rows ([G, n, >= max(ranks)], each group's first ranks[g] columns)."""
        G, n, _ = rows.shape
        b0, b1 = start // BLOCK, (start + n + BLOCK - 1) // BLOCK
        for g, r in enumerate(self.ranks):
            blk = self.group(g)[b:b + 1, :, b0:b1]
            cur = tiled_to_rows(blk.contiguous(), self.role)                        # [1, 1, (b1 - b0) * 32, r]
            cur[0, 0, start - b0 * BLOCK:start - b0 * BLOCK + n] = rows[g, :, :r].to(cur.dtype)
            blk.copy_(rows_to_tiled(cur, self.role))

    @property
    def shape(self) -> Tuple[int, int, int, int]:
        return (self.data.shape[0], len(self.ranks), self.max_seq, max(self.ranks))

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
