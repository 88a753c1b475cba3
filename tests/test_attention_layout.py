"""A CPU model of how attn_kernel (csrc/attention.hip) maps workgroups and waves to query rows and K/V tile sets.

Four-wave workgroups: block -> (batch, head, 128-row block); twelve-wave workgroups (every head of at least 384 query
rows): 384 consecutive rows of the (batch, head, row) range, each head's rows padded to Lq_pad (a multiple of 32).
The model restates the kernel's integer arithmetic and checks, over many shapes, that every stored (batch, head,
row) is computed by exactly one lane, that a wave's 32 rows lie in one head, that a workgroup spans at most two
heads with tile set c holding the K/V head the waves of set c read, that the copying waves cover both sets, and
that the XCD block remap is a permutation. Planted mistakes (the padding dropped, the head of the second set taken
from the first) fail it.
"""
import pytest

QB, FLAT_ROWS = 128, 384


def remap(blk, nblocks):
    return (blk % 8) * (nblocks // 8) + blk // 8 if nblocks % 8 == 0 else blk


def waves(B, H, Hkv, Lq, pad=True, second_from_first=False):
    """Yields (block, wave, b, h, q0, store, set, kv of set 0, kv of set 1, two) as the kernel computes them."""
    rep = H // Hkv
    if Lq >= FLAT_ROWS:
        lq_pad = (Lq + 31) // 32 * 32 if pad else Lq
        rows = B * H * lq_pad
        nblocks = (rows + FLAT_ROWS - 1) // FLAT_ROWS
        for block in range(nblocks):
            blk = remap(block, nblocks)
            g0 = blk * FLAT_ROWS
            bh0, bh1 = g0 // lq_pad, (min(g0 + FLAT_ROWS, rows) - 1) // lq_pad
            if second_from_first:
                bh1 = bh0
            kv = [(bh0 // H, (bh0 % H) // rep), (bh1 // H, (bh1 % H) // rep)]
            for wq in range(12):
                gw = g0 + 32 * wq
                store = gw < rows
                gc = gw if store else rows - 32
                bh = gc // lq_pad
                yield block, wq, bh // H, bh % H, gc % lq_pad, store, bh - bh0, kv[0], kv[1], bh1 != bh0
    else:
        qblocks = (Lq + QB - 1) // QB
        nblocks = qblocks * B * H
        for block in range(nblocks):
            blk = remap(block, nblocks)
            bh, qblk = divmod(blk, qblocks)
            for wq in range(4):
                kv = (bh // H, (bh % H) // rep)
                yield block, wq, bh // H, bh % H, qblk * QB + wq * 32, True, 0, kv, kv, False


def check(B, H, Hkv, Lq, **mistake):
    rep = H // Hkv
    seen = {}
    blocks = {}
    for block, wq, b, h, q0, store, st, kv0, kv1, two in waves(B, H, Hkv, Lq, **mistake):
        assert 0 <= b < B and 0 <= h < H and 0 <= st <= 1
        assert st == 0 or two, "a wave reads the second set only where the workgroup has one"
        # The set this wave reads holds its own (batch, KV head).
        assert (kv0, kv1)[st] == (b, h // rep), "wave reads another head's K/V"
        blocks.setdefault(block, set()).add((b, h))
        if not store:
            continue
        for lane_row in range(32):  # the wave's rows q0 .. q0 + 31, each stored only below Lq
            row = q0 + lane_row
            if row < Lq:
                key = (b, h, row)
                assert key not in seen, f"row {key} computed twice"
                seen[key] = (block, wq)
    assert len(seen) == B * H * Lq, "some rows not computed"
    assert all(len(heads) <= 2 for heads in blocks.values()), "a workgroup spans more than two heads"


SHAPES = [(1, 24, 24, 4096), (1, 2, 2, 384), (2, 3, 1, 416), (1, 4, 2, 640), (1, 3, 3, 400), (2, 2, 1, 1000), (1, 1, 1, 513),
          (3, 5, 5, 777), (1, 2, 2, 300), (2, 4, 1, 77), (1, 8, 2, 4160), (4, 6, 3, 1536)]


@pytest.mark.parametrize("B,H,Hkv,Lq", SHAPES)
def test_every_row_once_and_sets_match_heads(B, H, Hkv, Lq):
    check(B, H, Hkv, Lq)


@pytest.mark.parametrize("nblocks", [256, 264, 8, 7, 1000])
def test_block_remap_is_a_permutation(nblocks):
    assert sorted(remap(b, nblocks) for b in range(nblocks)) == list(range(nblocks))


def test_flat_configuration_is_one_round_of_whole_heads_per_xcd():
    """The attention configuration (24 heads x 4096 rows): 256 twelve-wave workgroups; XCD x (blocks x, x + 8, ...)
    covers 12288 consecutive rows, i.e. heads 3x .. 3x + 2."""
    heads_of_xcd = {}
    for block, wq, b, h, q0, store, st, kv0, kv1, two in waves(1, 24, 24, 4096):
        heads_of_xcd.setdefault(block % 8, set()).add(h)
    assert max(block for block, *_ in waves(1, 24, 24, 4096)) == 255
    assert all(heads == {3 * x, 3 * x + 1, 3 * x + 2} for x, heads in heads_of_xcd.items())


@pytest.mark.parametrize("mistake,shape", [({"pad": False}, (1, 3, 3, 400)), ({"second_from_first": True}, (2, 3, 1, 416)),
                                           ({"second_from_first": True}, (1, 4, 2, 640))])
def test_model_catches_mistakes(mistake, shape):
    with pytest.raises(AssertionError):
        check(*shape, **mistake)
