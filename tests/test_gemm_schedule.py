"""A CPU model of the copy / wait / barrier schedule of gemm8_kernel (csrc/gemm.hip), checked for races.

The kernel streams K in KT slices through NS LDS stages (slice s lives in stage s % NS). Each wave issues NI
asynchronous global->LDS copies per slice; `wait_copies_but<T>` retires its oldest copies until at most T are
outstanding (vmcnt counts loads in issue order); `__syncthreads` separates barrier epochs. The schedule:

  prologue: copy slices 0 .. NS-1 (those that exist); wait until (NS-1) NI remain if KT >= NS, else all; barrier;
            read the fragments of (slice 0, k step 0).
  slice kt (AHEAD = kt + NS < KT, MORE = kt + 1 < KT), k steps ks = 0 .. KS-1:
            at ks = KS-1 first: wait until (NS-2) NI remain if AHEAD, else all; barrier;
            products of (kt, ks); if AHEAD and ks = KS-1: copy slice kt + NS (into stage kt % NS);
            read the fragments of the next step: (kt, ks+1) if ks < KS-1, else (kt+1, 0) if MORE.

All waves run the same program, and two events of different waves are ordered only when a barrier separates
them. The model checks, for every wave pair at once:
  * a fragment read of slice s happens in a later epoch than the wait that retired all of s's copies (so after
    the barrier every wave's copies of s have landed), and the stage then holds s;
  * a copy into a stage is issued in a later epoch than every read of the slice that stage held before;
  * nothing reads or copies a slice that does not exist, and every slice is read.
A schedule mistake (copying one slice later than the stages allow, a wait threshold one slice too loose, the
barrier before the copies of the last k step dropped) fails one of these; test_model_catches_mistakes plants
each of them.

The W4A8 kernel (group-scaled, int4 weights, one W block per wave) runs a block-major slice of 16 products
instead: the A fragment of product P is read after product P - 3 (the first three of slice 0 in the prologue,
those of the next slice's first three after products 13-15), the next slice's packed W fragments after products 13
and 14, the wait and barrier sit before product 13, and the copies of slice kt + NS go out after products 13-15.
run_schedule_blockmajor models that order with the same checks.
"""
import pytest


def run_schedule(NS, KS, KT, NI=3, left=None, prologue_keep=None, copy_at=None, barrier_last=True):
    left = (NS - 2) * NI if left is None else left
    prologue_keep = ((NS - 1) * NI if KT >= NS else 0) if prologue_keep is None else prologue_keep
    copy_at = KS - 1 if copy_at is None else copy_at
    epoch = 0
    inflight = []  # slices of outstanding copies, in issue order
    landed_epoch = {}  # slice -> epoch of the wait that retired its last copy
    issued = {}  # slice -> number of copies issued
    holder = {}  # stage -> slice last copied into it
    last_read = {}  # slice -> epoch of its last fragment read
    errors = []

    def copy(s):
        if not 0 <= s < KT:
            errors.append(f"copy of missing slice {s}")
            return
        st = s % NS
        prev = holder.get(st)
        if prev is not None and last_read.get(prev, -1) >= epoch:
            errors.append(f"slice {s} copied into stage {st} in epoch {epoch} while slice {prev} is read there")
        holder[st] = s
        for _ in range(NI):
            inflight.append(s)
        issued[s] = issued.get(s, 0) + NI

    def wait(keep):
        while len(inflight) > keep:
            s = inflight.pop(0)
            if s not in inflight:
                landed_epoch[s] = epoch

    def barrier():
        nonlocal epoch
        epoch += 1

    def read(s):
        if not 0 <= s < KT:
            errors.append(f"read of missing slice {s}")
            return
        if landed_epoch.get(s, epoch) >= epoch or issued.get(s, 0) != NI:
            errors.append(f"slice {s} read in epoch {epoch} before its copies landed")
        if holder.get(s % NS) != s:
            errors.append(f"slice {s} read from stage {s % NS}, which holds slice {holder.get(s % NS)}")
        last_read[s] = epoch

    for s in range(min(NS, KT)):
        copy(s)
    wait(prologue_keep)
    barrier()
    read(0)
    for kt in range(KT):
        ahead, more = kt + NS < KT, kt + 1 < KT
        for ks in range(KS):
            if ks == KS - 1:
                wait(left if ahead else 0)
                if barrier_last:
                    barrier()
            if ahead and ks == copy_at:
                copy(kt + NS)
            if ks < KS - 1:
                read(kt)
            elif more:
                read(kt + 1)
    if set(last_read) != set(range(KT)):
        errors.append("not every slice was read")
    return errors


# (NS, KS): the kernel's configurations -- 128-byte slices (4 k steps) in 2 or 3 stages, 64-byte slices
# (2 k steps) in 4 stages -- plus neighbours.
@pytest.mark.parametrize("NS,KS", [(2, 4), (3, 4), (4, 2), (2, 2), (3, 2), (4, 4), (5, 2)])
@pytest.mark.parametrize("KT", list(range(1, 13)) + [24, 64])
def test_schedule_is_race_free(NS, KS, KT):
    assert run_schedule(NS, KS, KT) == []


@pytest.mark.parametrize("NS,KS", [(2, 4), (3, 4), (4, 2)])
def test_model_catches_mistakes(NS, KS):
    KT, NI = 10, 3
    # a wait that lets the next slice's copies stay in flight
    assert run_schedule(NS, KS, KT, NI, left=(NS - 1) * NI)
    # a prologue that does not wait for slice 0
    assert run_schedule(NS, KS, KT, NI, prologue_keep=NS * NI)
    # copies issued before the barrier of the last k step (the stage may still be read by another wave)
    assert run_schedule(NS, KS, KT, NI, copy_at=KS - 2)
    # the barrier before the last k step dropped
    assert run_schedule(NS, KS, KT, NI, barrier_last=False)


class Model:
    """Copies, waits, barriers and reads of the whole workgroup, with the race checks of run_schedule."""

    def __init__(self, NS, KT, NI):
        self.NS, self.KT, self.NI = NS, KT, NI
        self.epoch = 0
        self.inflight, self.landed, self.issued, self.holder, self.last_read, self.errors = [], {}, {}, {}, {}, []

    def copy(self, s, n):
        if not 0 <= s < self.KT:
            self.errors.append(f"copy of missing slice {s}")
            return
        st = s % self.NS
        prev = self.holder.get(st)
        if prev is not None and prev != s and self.last_read.get(prev, -1) >= self.epoch:
            self.errors.append(f"slice {s} copied into stage {st} in epoch {self.epoch} while slice {prev} is read there")
        self.holder[st] = s
        self.inflight += [s] * n
        self.issued[s] = self.issued.get(s, 0) + n

    def wait(self, keep):
        while len(self.inflight) > keep:
            s = self.inflight.pop(0)
            if s not in self.inflight:
                self.landed[s] = self.epoch

    def barrier(self):
        self.epoch += 1

    def read(self, s):
        if not 0 <= s < self.KT:
            self.errors.append(f"read of missing slice {s}")
            return
        if self.landed.get(s, self.epoch) >= self.epoch or self.issued.get(s, 0) != self.NI:
            self.errors.append(f"slice {s} read in epoch {self.epoch} before its copies landed")
        if self.holder.get(s % self.NS) != s:
            self.errors.append(f"slice {s} read from stage {s % self.NS}, which holds slice {self.holder.get(s % self.NS)}")
        self.last_read[s] = self.epoch


def run_schedule_blockmajor(NS, KT, NI=4, ahead_reads=3, barrier_at=13, copy_from=13, w_reads=(13, 14)):
    m = Model(NS, KT, NI)
    for s in range(min(NS, KT)):
        m.copy(s, NI)
    m.wait((NS - 1) * NI if KT >= NS else 0)
    m.barrier()
    m.read(0)  # the first products' A fragments and slice 0's packed W fragments
    copy_at = sorted({copy_from + c * (16 - copy_from) // NI for c in range(NI)})
    per = {p: sum(1 for c in range(NI) if copy_from + c * (16 - copy_from) // NI == p) for p in copy_at}
    for kt in range(KT):
        ahead, more = kt + NS < KT, kt + 1 < KT
        for P in range(16):
            if P == barrier_at:
                m.wait((NS - 2) * NI if ahead else 0)
                m.barrier()
            n = P + ahead_reads  # the A fragment read after product P
            if n < 16:
                m.read(kt)
            elif more:
                m.read(kt + 1)
            if more and P in w_reads:
                m.read(kt + 1)
            if ahead and P in per:
                m.copy(kt + NS, per[P])
    if set(m.last_read) != set(range(KT)):
        m.errors.append("not every slice was read")
    return m.errors


@pytest.mark.parametrize("NS", [3, 4])
@pytest.mark.parametrize("KT", list(range(1, 13)) + [24, 96])
def test_blockmajor_schedule_is_race_free(NS, KT):
    assert run_schedule_blockmajor(NS, KT) == []


@pytest.mark.parametrize("NS", [3, 4])
def test_blockmajor_model_catches_mistakes(NS):
    KT = 10
    # A fragments read only two products ahead: the read after product 13 is of this slice's stage, after the barrier
    assert run_schedule_blockmajor(NS, KT, ahead_reads=2)
    # the barrier one product later: the next slice's first A fragment is read before its copies are known to have landed
    assert run_schedule_blockmajor(NS, KT, barrier_at=14)
    # the copies of slice kt + NS issued before the barrier
    assert run_schedule_blockmajor(NS, KT, copy_from=12)


def tile_of(block, gx, gy, strips):
    """gemm8_kernel's block remap: block id -> (bx, by). Ids go round-robin to the 8 XCDs; XCD x takes the
    (gy / 2) x (gx / 4) sub-grid x, row by row, or (strips: the eight-wave W4A8 kernel, sub-grids at least 8 tiles wide)
    in strips four tiles tall, column by column."""
    by, bx = divmod(block, gx)
    if gx % 4 or gy % 2:
        return bx, by
    x, r, sx, sy = block % 8, block // 8, gx // 4, gy // 2
    if strips and sy % 4 == 0 and sx >= 8:
        strip, w = divmod(r, 4 * sx)
        return (x % 4) * sx + w // 4, (x // 4) * sy + strip * 4 + w % 4
    return (x % 4) * sx + r % sx, (x // 4) * sy + r // sx


@pytest.mark.parametrize("strips", [False, True])
@pytest.mark.parametrize("gx,gy", [(48, 32), (12, 16), (16, 16), (4, 8), (8, 4), (96, 32), (6, 3), (5, 8)])
def test_tile_order_is_a_permutation(gx, gy, strips):
    tiles = [tile_of(b, gx, gy, strips) for b in range(gx * gy)]
    assert sorted(tiles) == sorted((x, y) for x in range(gx) for y in range(gy))


def test_strip_order_groups_square_blocks():
    """With one block per CU (32 per XCD at a time), the first 32 tiles of an XCD span 4 rows x 8 columns."""
    gx, gy = 48, 32
    first = [tile_of(b, gx, gy, True) for b in range(0, 8 * 32, 8)]  # XCD 0's first 32 blocks
    assert len({y for _, y in first}) == 4 and len({x for x, _ in first}) == 8
