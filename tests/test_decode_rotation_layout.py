"""A CPU model of the ConvRot prologue of the fused decode GEMVs (rot_load / rot_to_lds in csrc/decode.hip).

The model restates the kernel's integer index arithmetic and its float32 operations in their order, thread by thread,
for the 512 (or 1024) threads of a workgroup: x is taken in sets of 16 consecutive values (set q = thread + NT r); the H4 steps
of stride 1 and 4 run on a set's registers; groups of 4 and 16 then write in reading order; larger groups write the
sets in the padded natural layout (word v + 4 (v >> 4) + 16 (v >> 8)), read them back transposed (thread u takes the
values 256 (u >> 4) + 16 i + (u & 15)), run the strides 16 and 64 in registers and, after every read, write in the
padded reading order (f4 j of lane l in step s at (4 s + j) 77 + l + 4 (l >> 4)). It checks, over K and group:
- every word written lies in the buffer the host sizes (rot_lds_bytes) and no two writes of a pass hit one word;
- the kernel's closed-form addresses equal the layout functions they stand for;
- the LDS banks (64 x 4 bytes) of each pass: a wave's transposed reads and reading-order writes touch 64 distinct
  banks, and its 16-lane groups of 16-byte accesses (natural writes, product reads) 16 distinct 16-byte bank groups;
- the buffer read back in reading order equals the oracle's rotation bit for bit.
Planted mistakes (the transposed base off by one block, the stride-4 step skipped, the half step's lane order
dropped, an even row length) fail it.

It also models rotate_group_kernel (rda_rotate, any group of 4^n up to 16384): the group in padded LDS (word
p + p / 16), one pass per base-16 digit of the value index with each thread's sets of 16 (or 4) values in registers;
each pass's sets partition the group, the words stay in the host's LDS size, and the result is the oracle's rotation.
"""
import numpy as np
import pytest

import oracle

NT, RO_ROW = 512, 77


def nat_word(v):
    return v + 4 * (v >> 4) + 16 * (v >> 8)


def ro_f4(s, j, l, row=RO_ROW):
    return (4 * s + j) * row + l + 4 * (l >> 4)


def ro_of_value(v, steps, row=RO_ROW):
    if v < steps * 1024:
        return ro_f4(v >> 10, (v >> 2) & 3, (v >> 4) & 63, row)
    t = v - steps * 1024
    return ro_f4(steps, (t >> 2) & 1, t >> 3, row)


def rot_lds_words(K):
    rows = 4 * (K // 1024) + (2 if K % 1024 else 0)
    return max(K + K // 4 + K // 16, 4 * rows * RO_ROW)


def h4(a, b, c, d):
    s = a + b + c + d  # float32, left to right
    two = np.float32(2)
    return s - two * d, s - two * c, s - two * b, s - two * a


def check_banks(words, per_group, what):
    """words[lane] for one instruction of one wave: each group of `per_group` lanes must hit distinct banks."""
    for g0 in range(0, len(words), per_group):
        grp = [w for w in words[g0:g0 + per_group] if w is not None]
        if per_group == 64:
            banks = [w % 64 for w in grp]
        else:  # 16-byte accesses: 16 bank groups of 4 words
            banks = [(w // 4) % 16 for w in grp]
        assert len(set(banks)) == len(banks), f"{what}: bank conflict {sorted(banks)}"


def rot_to_lds(x, K, group, mistake=None, NT=NT):
    """The LDS buffer (float32 words) that rot_to_lds leaves for the products, and its reading-order read-back."""
    steps, sets = K // 1024, K // 16
    rs = (sets + NT - 1) // NT
    row = 76 if mistake == "row" else RO_ROW
    size = rot_lds_words(K)
    xw = np.full(size, np.nan, np.float32)
    norm = np.float32(1) / np.sqrt(np.float32(group))

    def ro(v):
        if mistake == "tail" and v >= steps * 1024:
            return ro_f4(steps, 0, 0, row) + (v - steps * 1024) // 4
        return ro_of_value(v, steps, row)

    regs = {}
    for t in range(NT):
        for r in range(rs):
            q = t + NT * r
            src = 16 * (q if q < sets else 0)
            regs[t, r] = [x[src + 4 * j:src + 4 * j + 4].astype(np.float32).copy() for j in range(4)]
    for v in regs.values():
        for j in range(4):
            v[j] = np.array(h4(*v[j]), np.float32)  # stride 1
        if group >= 16 and mistake != "skip4":
            v[0], v[1], v[2], v[3] = h4(*v)  # stride 4
    if group <= 16:
        written = set()
        for (t, r), v in regs.items():
            q = t + NT * r
            if q < sets:
                for j in range(4):
                    f = ro(16 * q + 4 * j)
                    for e in range(4):
                        assert 4 * f + e < size and 4 * f + e not in written
                        written.add(4 * f + e)
                        xw[4 * f + e] = v[j][e] * norm
        return xw
    # natural writes (f4s), with the kernel's closed form and its banks
    written = set()
    for r in range(rs):
        for j in range(4):
            for w0 in range(0, NT, 64):
                lanes = []
                for t in range(w0, w0 + 64):
                    q = t + NT * r
                    if q < sets:
                        a = 20 * q + 16 * (q >> 4) + 4 * j
                        assert a == nat_word(16 * q + 4 * j)
                        lanes.append(a)
                        for e in range(4):
                            assert a + e < size and a + e not in written
                            written.add(a + e)
                            xw[a + e] = regs[t, r][j][e]
                    else:
                        lanes.append(None)
                check_banks(lanes, 16, "natural write")
    # transposed reads
    y = {}
    for r in range(rs):
        for w0 in range(0, NT, 64):
            for i in range(16):
                lanes = []
                for t in range(w0, w0 + 64):
                    u = t + NT * r
                    if u < sets:
                        b = u >> 4
                        base = 336 * b + (u & 15) + (336 if mistake == "base" else 0)
                        a = base + 20 * i
                        assert mistake == "base" or a == nat_word(256 * b + 16 * i + (u & 15))
                        assert 0 <= a < size, "read outside the buffer"
                        lanes.append(a)
                        y.setdefault((t, r), [None] * 16)[i] = np.float32(xw[a])
                    else:
                        lanes.append(None)
                check_banks(lanes, 64, "transposed read")
    for yy in y.values():
        for k in range(4):
            yy[4 * k], yy[4 * k + 1], yy[4 * k + 2], yy[4 * k + 3] = h4(yy[4 * k], yy[4 * k + 1], yy[4 * k + 2], yy[4 * k + 3])
        if group >= 256:
            for m in range(4):
                yy[m], yy[m + 4], yy[m + 8], yy[m + 12] = h4(yy[m], yy[m + 4], yy[m + 8], yy[m + 12])
    # reading-order writes after every read
    written = set()
    for r in range(rs):
        for w0 in range(0, NT, 64):
            for i in range(16):
                lanes = []
                for t in range(w0, w0 + 64):
                    u = t + NT * r
                    if u < sets:
                        b, p = u >> 4, u & 15
                        if b < 4 * steps:
                            a = 4 * ((4 * (b >> 2) + (p >> 2)) * row + 20 * (b & 3)) + (p & 3) + 4 * i
                        else:
                            a = 4 * ((4 * steps + ((p >> 2) & 1)) * row + 40 * (b - 4 * steps) + (p >> 3)) + (p & 3) + 8 * i + 16 * (i >> 3)
                        val = 256 * b + 16 * i + p
                        if mistake != "tail":
                            assert a == 4 * ro(val & ~3) + (val & 3)
                        else:
                            a = 4 * ro(val & ~3) + (val & 3)
                        assert 0 <= a < size and a not in written, "reading-order write outside the buffer or twice"
                        written.add(a)
                        lanes.append(a)
                        xw[a] = y[t, r][i] * norm
                    else:
                        lanes.append(None)
                if not any(256 * ((t + NT * r) >> 4) >= 1024 * steps for t in range(w0, w0 + 64) if t + NT * r < sets):
                    check_banks(lanes, 64, "reading-order write")
    return xw


def read_back(xw, K, row=RO_ROW):
    """x as the products read it: lane l's f4 j of step s from ro_f4(s, j, l); also checks their banks."""
    steps = K // 1024
    out = np.empty(K, np.float32)
    for s in range(steps + (1 if K % 1024 else 0)):
        for j in range(4 if s < steps else 2):
            lanes = [4 * ro_f4(s, j, l, row) for l in range(64)]
            check_banks(lanes, 16, "product read")
            for l in range(64):
                v = s * 1024 + (16 * l + 4 * j if s < steps else 8 * l + 4 * j)
                out[v:v + 4] = xw[lanes[l]:lanes[l] + 4]
    return out


CASES = [(1024, 4), (1024, 16), (1024, 64), (1024, 256), (4096, 256), (4096, 64), (1536, 256), (512, 64), (512, 256),
         (2560, 16), (12288, 256), (16384, 256), (9728, 256), (15872, 64), (8192, 256)]


@pytest.mark.parametrize("K,group,nt", [(K, g, 512) for K, g in CASES] + [(12288, 256, 1024), (16384, 64, 1024), (9216, 16, 1024)])
def test_rotation_layout_matches_oracle(K, group, nt):
    """512 threads (eight waves) everywhere; 1024 (sixteen waves) for rows past 8192 values."""
    x = np.random.default_rng(K + group).standard_normal(K).astype(np.float32)
    got = read_back(rot_to_lds(x, K, group, NT=nt), K)
    ref = oracle.rotate_f32(x.reshape(-1, group), group).reshape(-1)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("mistake,K,group", [("base", 4096, 256), ("skip4", 1024, 64), ("tail", 1536, 256), ("row", 4096, 256)])
def test_model_catches_mistakes(mistake, K, group):
    x = np.random.default_rng(7).standard_normal(K).astype(np.float32)
    with pytest.raises(AssertionError):
        xw = rot_to_lds(x, K, group, mistake=mistake)
        ref = oracle.rotate_f32(x.reshape(-1, group), group).reshape(-1)
        assert np.array_equal(read_back(xw, K, 76 if mistake == "row" else RO_ROW).view(np.uint32), ref.view(np.uint32))


# ------------------------------------------------------------------ rotate_group_kernel (rda_rotate), any group of 4^n

def rot_word(p):
    return p + (p >> 4)


def h4_step(a, b, c, d):
    """The kernel's h4_step on float32 values: sum = ((a + b) + c) + d, then sum - 2 d, sum - 2 c, sum - 2 b, sum - 2 a."""
    f = np.float32
    s = f(f(f(a + b) + c) + d)
    return f(s - f(2) * d), f(s - f(2) * c), f(s - f(2) * b), f(s - f(2) * a)


def rotate_group_model(x, group, threads=256):
    """rotate_group_kernel for one group, thread by thread and pass by pass: returns (output, LDS words touched per
    pass as lists of (thread, word, is_write))."""
    words = rot_word(group - 1) + 1
    lds = np.full(words, np.nan, np.float32)
    for p in range(group):
        lds[rot_word(p)] = x[p]
    digits = (group.bit_length() - 1) // 2
    passes, k, span = [], 0, 1
    while 2 * k < digits:
        W = 16 if 2 * k + 1 < digits else 4
        touched, new = [], lds.copy()
        for t in range(threads):
            for q in range(t, group // W, threads):
                lo, hi = q % span, q // span
                first = hi * W * span + lo
                idx = [rot_word(first + j * span) for j in range(W)]
                v = [lds[i] for i in idx]
                if W == 16:
                    for b in range(0, 16, 4):
                        v[b:b + 4] = h4_step(*v[b:b + 4])
                    for m in range(4):
                        v[m], v[m + 4], v[m + 8], v[m + 12] = h4_step(v[m], v[m + 4], v[m + 8], v[m + 12])
                else:
                    v = list(h4_step(*v))
                for i, val in zip(idx, v):
                    new[i] = val
                touched += [(t, i) for i in idx]
        passes.append(touched)
        lds = new
        k, span = k + 1, span * 16
    norm = np.float32(1) / np.sqrt(np.float32(group))
    out = np.array([np.float32(lds[rot_word(p)] * norm) for p in range(group)], np.float32)
    return out, passes, words


@pytest.mark.parametrize("group", [4, 16, 64, 256, 1024, 4096, 16384])
def test_rotate_group_kernel_model(group):
    """Each pass's sets partition the group (every value read and written once, by one thread), every word lies in the
    host's LDS size (rot_word(group) words), a wave's first-value reads of a pass fall in distinct banks (up to 2-way
    in the stride-256 pass), and the result equals the oracle's rotation bit for bit."""
    rng = np.random.default_rng(group)
    x = (rng.standard_normal(group) * 3).astype(np.float32)
    out, passes, words = rotate_group_model(x, group)
    assert words <= rot_word(group)
    assert len(passes) == ((group.bit_length() - 1) // 2 + 1) // 2
    for touched in passes:
        ws = [w for _, w in touched]
        assert len(ws) == group and len(set(ws)) == group and max(ws) < words
        first_reads = {}
        for t, w in touched:
            first_reads.setdefault(t, w)  # a thread's first word of the pass: lanes of a wave read it together
        for wave in range(0, 256, 64):
            banks = [first_reads[t] % 64 for t in range(wave, wave + 64) if t in first_reads]
            if banks:
                assert max(np.bincount(banks)) <= 2
    ref = oracle.rotate_f32(x.reshape(1, group), group).reshape(-1)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_rotate_group_model_sees_a_skipped_step():
    """The model is not vacuous: dropping the stride-4 step of the first pass changes the result."""
    x = np.random.default_rng(1).standard_normal(256).astype(np.float32)
    global h4_step
    saved = h4_step
    calls = []

    def skip_second(a, b, c, d):
        calls.append(1)
        return (a, b, c, d) if len(calls) == 5 else saved(a, b, c, d)

    h4_step = skip_second
    try:
        out, _, _ = rotate_group_model(x, 256)
    finally:
        h4_step = saved
    assert not np.array_equal(out, oracle.rotate_f32(x.reshape(1, 256), 256).reshape(-1))
