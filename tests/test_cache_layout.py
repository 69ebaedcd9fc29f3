"""Tiled latent-cache layout: round trip and the slot -> (position, width index) mapping the kernel reads."""
import pytest
import torch

from palu_tt.cache import GroupedLatentCache, LatentCache, rows_to_tiled, tiled_to_rows


@pytest.mark.parametrize("role", ["k", "v"])
@pytest.mark.parametrize("S,r", [(32, 32), (64, 64), (256, 96), (96, 128), (64, 48), (32, 80), (96, 112), (32, 16)])
def test_round_trip_is_exact(S, r, role):
    rows = torch.randn(2, 3, S, r).to(torch.bfloat16)
    tiled = rows_to_tiled(rows, role)
    assert tiled.shape == (2, 3, S // 32, r // 16, 64, 8)
    assert torch.equal(tiled_to_rows(tiled, role), rows)


def test_slot_mapping_matches_the_documented_operand_order():
    """Tile (c, kb), slot l = 16*g + n holds r-index 32*kb + 8*g + j of position 32*blk + 8*(n//4) + 4*c + n%4."""
    S, r = 64, 64
    pos = torch.arange(S)[:, None].expand(S, r)
    col = torch.arange(r)[None, :].expand(S, r)
    code = (pos * 1000 + col).float()[None, None]          # exact in fp32
    tiled = rows_to_tiled(code, "k")
    for blk in range(S // 32):
        for c in range(2):
            for kb in range(r // 32):
                for l in range(64):
                    g, n = divmod(l, 16)
                    p = 32 * blk + 8 * (n // 4) + 4 * c + n % 4
                    for j in range(8):
                        assert tiled[0, 0, blk, c * (r // 32) + kb, l, j] == p * 1000 + 32 * kb + 8 * g + j


@pytest.mark.parametrize("r", [48, 80])
def test_k_half_tile_slot_mapping(r):
    """K width an odd multiple of 16: half-block c of a block is 16 r elements from c * 16 r; its full tiles
    keep the 32-deep order and its last 256 elements hold r-indices 32 (r // 32) + 4 g + j (j < 4) of
    position 8 (n // 4) + 4 c + n % 4 in slot 16 g + n."""
    S = 64
    kbf = r // 32
    pos = torch.arange(S)[:, None].expand(S, r)
    col = torch.arange(r)[None, :].expand(S, r)
    flat = rows_to_tiled((pos * 1000 + col).float()[None, None], "k").reshape(S // 32, 32 * r)
    for blk in range(S // 32):
        for c in range(2):
            for l in range(64):
                g, n = divmod(l, 16)
                p = 32 * blk + 8 * (n // 4) + 4 * c + n % 4
                for kb in range(kbf):
                    for j in range(8):
                        assert flat[blk, c * 16 * r + kb * 512 + 8 * l + j] == p * 1000 + 32 * kb + 8 * g + j
                for j in range(4):
                    assert flat[blk, c * 16 * r + kbf * 512 + 4 * l + j] == p * 1000 + 32 * kbf + 4 * g + j


def test_v_slot_mapping_matches_the_documented_operand_order():
    """V order: tile mt, slot l = 16*g + m holds positions 32*blk + 8*g + j (j < 8) of r-index 16*mt + m."""
    S, r = 64, 64
    pos = torch.arange(S)[:, None].expand(S, r)
    col = torch.arange(r)[None, :].expand(S, r)
    tiled = rows_to_tiled((pos * 1000 + col).float()[None, None], "v")
    for blk in range(S // 32):
        for mt in range(r // 16):
            for l in range(64):
                g, m = divmod(l, 16)
                for j in range(8):
                    assert tiled[0, 0, blk, mt, l, j] == (32 * blk + 8 * g + j) * 1000 + 16 * mt + m


def test_latent_cache_reports_logical_shape():
    lc = LatentCache.zeros(2, 8, 128, 64, device="cpu", role="v")
    assert lc.shape == (2, 8, 128, 64) and lc.dtype == torch.bfloat16 and lc.role == "v"
    assert lc.nbytes() == 2 * 8 * 128 * 64 * 2
    rows = torch.randn(2, 8, 128, 64).to(torch.bfloat16)
    for role in ("k", "v"):
        assert torch.equal(LatentCache.from_rows(rows, role).to_rows(), rows)


@pytest.mark.parametrize("role", ["k", "v"])
def test_grouped_cache_stores_each_group_at_its_own_ranks(role):
    """Row b's group streams lie one after another, group g from S * (ranks before it), each the tiled
    storage of that group's first ranks[g] columns; to_rows pads with zeros; write_rows touches only
    each group's own columns."""
    B, S, ranks = 2, 64, (32, 96, 64)
    rows = torch.randn(B, 3, S, 96).to(torch.bfloat16)
    c = GroupedLatentCache.from_rows(rows, ranks, role)
    assert c.data.shape == (B, S * sum(ranks)) and c.shape == (B, 3, S, 96)
    off = 0
    for g, r in enumerate(ranks):
        for b in range(B):
            assert torch.equal(c.data[b, off:off + S * r], rows_to_tiled(rows[b:b + 1, g:g + 1, :, :r].contiguous(), role).flatten())
        off += S * r
    exp = rows.clone()
    for g, r in enumerate(ranks):
        exp[:, g, :, r:] = 0
    assert torch.equal(c.to_rows(), exp)
    new = torch.randn(3, 5, 96).to(torch.bfloat16)
    c.write_rows(1, 30, new)
    for g, r in enumerate(ranks):
        exp[1, g, 30:35, :r] = new[g, :, :r]
    assert torch.equal(c.to_rows(), exp)
