"""The KV-cache block layout (include/ssd_mi355x.h, csrc/common.h k_off / v_off): a bijection
of a (layer, kv head) region, K tiles that hold 8 consecutive dims of one slot per lane, V tiles
that hold 8 consecutive slots of one dim per lane, and kv_tile / kv_untile inverting each other.
CPU only."""

import pytest
import torch


def _ops():
    from ssd import ops
    return ops


@pytest.mark.parametrize("cap,hd", [(64, 32), (128, 64), (192, 128)])
def test_block_index_is_a_permutation(cap, hd):
    k_idx, v_idx = _ops().kv_block_index(cap, hd, "cpu")
    for idx in (k_idx, v_idx):
        assert idx.shape == (cap, hd)
        assert torch.equal(idx.reshape(-1).sort().values, torch.arange(cap * hd))


@pytest.mark.parametrize("hd", [32, 64, 128])
def test_tiles_follow_the_mfma_operand_lanes(hd):
    """K tile (kt, ks) lane g*16+i = slot key(kt, i) dims 32ks+8g..+8; V tile (dt, c) lane g*16+i =
    slots 32c+8g..+8 of dim 16dt+i -- checked from the offsets, for every slot of two blocks."""
    cap = 128
    k_idx, v_idx = _ops().kv_block_index(cap, hd, "cpu")
    KS, DT = hd // 32, hd // 16
    for s in range(cap):
        b, o = divmod(s, 64)
        kt, i = (o // 32) * 2 + (o // 4) % 2, ((o // 8) % 4) * 4 + o % 4
        # the inverse of the attention kernel's key order within a tile
        assert (kt // 2) * 32 + (i // 4) * 8 + (kt % 2) * 4 + i % 4 == o
        for d in range(0, hd, 8):
            ks, g = d // 32, (d // 8) % 4
            tile = (b * 4 + kt) * KS + ks
            assert k_idx[s, d].item() == (tile * 64 + g * 16 + i) * 8
            assert torch.equal(k_idx[s, d:d + 8], k_idx[s, d] + torch.arange(8))
        for d in range(hd):
            c, g = o // 32, (o // 8) % 4
            tile = (b * DT + d // 16) * 2 + c
            assert v_idx[s, d].item() == (tile * 64 + g * 16 + d % 16) * 8 + o % 8


def test_tile_untile_round_trip_and_cache_update():
    from ssd.engine.kv_cache import KVCache

    ops = _ops()
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 2, 128, 64, generator=g).to(torch.bfloat16)
    for which in ("k", "v"):
        t = ops.kv_tile(x, which)
        assert t.shape == (3, 2, 128 * 64)
        assert torch.equal(ops.kv_untile(t, 128, 64, which), x)
    cache = KVCache(2, 100, 2, 64, "cpu")
    assert cache.capacity == 128
    k = torch.randn(1, 2, 7, 64, generator=g)
    v = torch.randn(1, 2, 7, 64, generator=g)
    kk, vv = cache.update(1, k, v)
    assert torch.equal(kk[0], k[0].to(torch.bfloat16)) and torch.equal(vv[0], v[0].to(torch.bfloat16))
    cache.advance(7)
    k2 = torch.randn(1, 2, 3, 64, generator=g)
    kk, vv = cache.update(1, k2, k2)
    assert torch.equal(kk[0, :, :7], k[0].to(torch.bfloat16)) and torch.equal(kk[0, :, 7:], k2[0].to(torch.bfloat16))
    assert cache.k[0].abs().sum() == 0
