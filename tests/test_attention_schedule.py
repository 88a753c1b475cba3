"""A CPU model of the fp16 tile loop of attn_kernel (csrc/attention.hip): where each tile's exponentials, lazy-rescale
check (settle) and PV products run, checked for the data each of them needs.

A tile's P is made in eight parts of two exponential pairs: parts 0-3 (keys 0-15, the P operand of the first four PV
products) and parts 4-7 (keys 16-31, the last four). The kernel's order, restated from its `step` lambda and the
prologue: tile 0's scores, then its parts 0-3 into pf[0]; step i (not the last): the score products of tile i + 1
with tile i's parts 4-7 beside products 1, 3, 5, 7; settle(i); l_old = l; tile i's PV products, tile i + 1's parts
0-3 (into registers pn) beside PV products 1, 3 of each half; pf[0] = pn. The last step: tile i's parts 4-7,
settle(i), its PV products.

The checks, per tile t:
  * settle(t) sees l grown by exactly tile t's eight parts, in part order, since its l_old (so the fast-path test
    l <= l_old + 64 and the slow path's restart from l_old are the rule's), and every part of t ran before it;
  * every part of t ran with the running maximum as settle(t - 1) left it (one m for the whole tile);
  * the P operand each PV product of t reads holds t's parts for its keys: no part of tile t + 1 has overwritten it;
  * l sums the tiles in order.
Planted mistakes (parts 0-3 of the next tile written straight into pf[0] beside the first PV products; l_old taken at
the start of the step; tile i's last parts after settle(i)) each fail one check (test_model_catches_mistakes).
"""
import pytest


def run(tiles, pn_buffer=True, l_old_at_start=False, late_parts=False):
    regs = {"pf0": None, "pf1": None, "pn": None}  # (tile, parts) each P register set holds
    l_log = []  # (tile, part) in the order l accumulates them
    m_version = 0  # settles done
    part_m = {}
    errors = []
    l_old_mark = 0

    def part(t, k, dest):
        part_m[(t, k)] = m_version
        l_log.append((t, k))
        cur = regs[dest]
        if cur is None or cur[0] != t:
            regs[dest] = (t, {k})
        else:
            cur[1].add(k)

    def settle(t, mark):
        nonlocal m_version
        grown = l_log[mark:]
        if grown != [(t, k) for k in range(8)]:
            errors.append(f"settle({t}) sees l grown by {grown}")
        m_version += 1

    def pv_read(t, reg, keys):
        held = regs[reg]
        if held is None or held[0] != t or held[1] != keys:
            errors.append(f"PV of tile {t} reads {reg} holding {held}, not parts {sorted(keys)}")

    def pv(t, hook2_parts, hook_target):
        # first four products read P keys 0-15, the last four keys 16-31; hooks after products 1 and 3 of each half
        for half, reg, keys in ((0, "pf0", {0, 1, 2, 3}), (1, "pf1", {4, 5, 6, 7})):
            for dt in range(4):
                pv_read(t, reg, keys)
                if dt & 1 and hook2_parts is not None:
                    hook2_parts(2 * half + (dt >> 1), hook_target)

    # prologue: tile 0's scores, parts 0-3
    for k in range(4):
        part(0, k, "pf0")
    for i in range(tiles):
        if l_old_at_start:
            l_old_mark = len(l_log)
        if i < tiles - 1:
            if not late_parts:
                for k in range(4, 8):  # beside score products 1, 3, 5, 7 of tile i + 1
                    part(i, k, "pf1")
            settle(i, l_old_mark)
            if late_parts:
                for k in range(4, 8):
                    part(i, k, "pf1")
            if not l_old_at_start:
                l_old_mark = len(l_log)
            target = "pn" if pn_buffer else "pf0"
            pv(i, lambda k, dest, nxt=i + 1: part(nxt, k, dest), target)
            if pn_buffer:
                regs["pf0"] = regs["pn"]
        else:
            for k in range(4, 8):
                part(i, k, "pf1")
            settle(i, l_old_mark)
            pv(i, None, None)
    for t in range(tiles):
        for k in range(8):
            if part_m.get((t, k)) != t:
                errors.append(f"part {k} of tile {t} ran after {part_m.get((t, k))} settles, not {t}")
    if l_log != [(t, k) for t in range(tiles) for k in range(8)]:
        errors.append("l does not sum the tiles in order")
    return errors


@pytest.mark.parametrize("tiles", [1, 2, 3, 7, 8, 13, 128])
def test_schedule(tiles):
    assert run(tiles) == []


@pytest.mark.parametrize("mistake", [dict(pn_buffer=False), dict(l_old_at_start=True), dict(late_parts=True)])
def test_model_catches_mistakes(mistake):
    assert run(8, **mistake) != []
