"""Writes gemm2_loop.inc: the per-block body of k_gemm2_q8's main loop (prefill.hip), a fixed schedule of LDS fragment
reads, int8 MFMAs and VALU steps.

The LDS reads are inline asm (the compiler cannot see which direct-to-LDS load fills which stage), so every use of a
read's result must follow an explicit `s_waitcnt lgkmcnt(N)` naming it.  N depends on how many reads were issued after
it; this script tracks the issue order and computes each N, so an edit of the schedule cannot leave a wrong count.
Run it after editing:  python3 gen_gemm2_loop.py > gemm2_loop.inc

One 128-column block: K = 4 steps of 32; the wave's 64 x 64 tile is rows mi0 / mi1 x tokens ni0 / ni1, one int32
accumulator T[mi][ni] each; A0 / A1 hold the block's weight fragments of rows mi0 / mi1 from the hi plane to the lo
plane.  Four quarters of 8 MFMAs, each paired with VALU work that does not depend on its own MFMAs:
  Q1  hi plane of rows mi0       || the previous block's fp32 step of rows mi1: acc = fma(bs, (float) T, acc) (64 VALU)
  Q2  hi plane of rows mi1       || shift-add of rows mi0: T = 256 T + 128 sum(W) (32 VALU)
  Q3  lo plane of rows mi0       || shift-add of rows mi1 (32 VALU)
  Q4  lo plane of rows mi1       || fp32 step of rows mi0 (64 VALU)
Reads run LOOK steps ahead of the MFMAs (token fragments cycle through LOOK + 1 register pairs); each quarter's row
sums / token scales are read just before its first step.
"""
import sys

LOOK = 2

out = []
issued = []   # LDS reads in flight, oldest first


def emit(s):
    out.append("    " + s)


def read(name, expr):
    issued.append(name)
    emit(f"{name} = {expr};")


def wait(*names):
    """wait until the reads named (and all issued before them) have landed; name every register that lands"""
    global issued
    idx = max(len(issued) - 1 - issued[::-1].index(n) for n in names)
    done, issued = issued[:idx + 1], issued[idx + 1:]
    assert len(issued) + len(done) <= 15
    regs = ", ".join(f'"+v"({r})' for r in dict.fromkeys(done))
    emit(f'asm volatile("s_waitcnt lgkmcnt({len(issued)})" : {regs});')


def RA(ks, mi):
    return f"lds_read16o<{mi * 4096}>(st + ra[{ks}])"


def RB(plane, ks, ni):
    base = "kG2XH" if plane == "h" else "kG2XL"
    return f"lds_read16o<{base} + {ni * 4096}>(st + rb[{ks}])"


def fp32_step(t, half, bs):
    for i in range(8 * half, 8 * half + 8):
        emit(f"acc[{t[1]}][{t[2]}][{i}] = __builtin_fmaf({bs}, (float)T[{t[1]}][{t[2]}][{i}], acc[{t[1]}][{t[2]}][{i}]);")


def shift_add(t, w):
    for i in range(16):
        emit(f"T[{t[1]}][{t[2]}][{i}] = T[{t[1]}][{t[2]}][{i}] * 256 + {w}{i // 4}[{i % 4}];")


class Quarter:
    def __init__(self, title, mi, plane, read_a, valu, extras):
        self.title, self.mi, self.plane, self.read_a, self.valu, self.extras = title, mi, plane, read_a, valu, extras


def valu_q1(ks):
    # at the first block T and the scales are zero: acc + 0 * 0 = acc, no branch needed
    fp32_step("T10" if ks < 2 else "T11", ks % 2, "pb0" if ks < 2 else "pb1")


def valu_q2(ks):
    if ks < 2:
        shift_add(("T00", "T01")[ks], "w")


def valu_q3(ks):
    if ks < 2:
        shift_add(("T10", "T11")[ks], "x")


def valu_q4(ks):
    fp32_step("T00" if ks < 2 else "T01", ks % 2, "nb0" if ks < 2 else "nb1")


def extras_ws(mi, reg):
    def f():
        for j in range(4):
            read(f"{reg}{j}", f"lds_read16o<{128 * mi + 32 * j}>(st + rws)")
    return f


def extras_bs():
    read("nb0", "lds_read4o<0>(st + rbs)")
    read("nb1", "lds_read4o<128>(st + rbs)")


quarters = [
    Quarter("Q1: hi plane of rows mi0 || the previous block's fp32 step of rows mi1", 0, "h", True, valu_q1, None),
    Quarter("Q2: hi plane of rows mi1 || shift-add of rows mi0", 1, "h", True, valu_q2, extras_ws(0, "w")),
    Quarter("Q3: lo plane of rows mi0 || shift-add of rows mi1", 0, "l", False, valu_q3, extras_ws(1, "x")),
    Quarter("Q4: lo plane of rows mi1 || fp32 step of rows mi0", 1, "l", False, valu_q4, extras_bs),
]


def schedule_halves():
    """the four quarters above: 8 MFMAs on one row half per step pair; token fragments read once per row half"""
    steps = [(q, ks) for q in quarters for ks in range(4)]
    bset = [f"f{i}" for i in range(LOOK + 1)]

    def regs_of(i):
        q, ks = steps[i]
        s_ = bset[i % (LOOK + 1)]
        return f"A{q.mi}[{ks}]", f"{s_}a", f"{s_}b"

    def issue_step(i):
        q, ks = steps[i]
        if ks == 0 and q.extras:
            q.extras()
        a, b0, b1 = regs_of(i)
        if q.read_a:
            read(a, RA(ks, q.mi))
        read(b0, RB(q.plane, ks, 0))
        read(b1, RB(q.plane, ks, 1))

    for i in range(LOOK):
        issue_step(i)
    for i, (q, ks) in enumerate(steps):
        if ks == 0:
            emit(f"// ---- {q.title}")
        if i + LOOK < len(steps):
            issue_step(i + LOOK)
        a, b0, b1 = regs_of(i)
        wait(*((a,) if q.read_a else ()), b0, b1)
        t0, t1 = f"T[{q.mi}][0]", f"T[{q.mi}][1]"
        first = q.plane == "h" and ks == 0
        emit(f"{t0} = __builtin_amdgcn_mfma_i32_32x32x32_i8({a}, {b0}, {'zero' if first else t0}, 0, 0, 0);")
        emit(f"{t1} = __builtin_amdgcn_mfma_i32_32x32x32_i8({a}, {b1}, {'zero' if first else t1}, 0, 0, 0);")
        q.valu(ks)


def schedule_steps():
    """4 MFMAs (all four tiles) per step, every fragment read once per plane (A held from hi to lo); the VALU steps
    staggered by tile pair: the shift-add of row half mi0 under the last hi MFMAs of mi1 and the first lo MFMAs, the
    fp32 step of mi0 under the last lo MFMAs of mi1, that of mi1 under the next block's first hi MFMAs"""
    LOOK = 1   # a step is 4 MFMAs; two steps of reads (16) would pass the 15-read limit with the row sums
    steps = [("h", ks) for ks in range(4)] + [("l", ks) for ks in range(4)]
    bset = [f"f{i}" for i in range(LOOK + 1)]

    def issue_step(i):
        plane, ks = steps[i]
        if i == 4:
            extras_ws(0, "w")()
            extras_ws(1, "x")()
        if i == 7:
            extras_bs()
        s_ = bset[i % (LOOK + 1)]
        if plane == "h":
            read(f"A0[{ks}]", RA(ks, 0)); read(f"A1[{ks}]", RA(ks, 1))
        read(f"{s_}a", RB(plane, ks, 0)); read(f"{s_}b", RB(plane, ks, 1))

    for i in range(LOOK):
        issue_step(i)
    for i, (plane, ks) in enumerate(steps):
        if i + LOOK < len(steps):
            issue_step(i + LOOK)
        s_ = bset[i % (LOOK + 1)]
        b0, b1 = f"{s_}a", f"{s_}b"
        wait(*((f"A0[{ks}]", f"A1[{ks}]") if plane == "h" else ()), b0, b1)
        first = plane == "h" and ks == 0
        for mi in (0, 1):
            if plane == "l" and ks == 0:   # the shift-add of this row half just before its first lo MFMAs
                shift_add(f"T{mi}0", "w" if mi == 0 else "x")
                shift_add(f"T{mi}1", "w" if mi == 0 else "x")
            for ni, b in ((0, b0), (1, b1)):
                t = f"T[{mi}][{ni}]"
                emit(f"{t} = __builtin_amdgcn_mfma_i32_32x32x32_i8(A{mi}[{ks}], {b}, {'zero' if first else t}, 0, 0, 0);")
            if plane == "h" and ks == 0 and mi == 0:   # the previous block's fp32 step of mi1 before its first hi MFMA
                for half in (0, 1):
                    fp32_step("T10", half, "pb0")
                for half in (0, 1):
                    fp32_step("T11", half, "pb1")
        if plane == "l" and ks == 3:   # this block's fp32 step of mi0 under the last MFMAs of mi1
            for half in (0, 1):
                fp32_step("T00", half, "nb0")
            for half in (0, 1):
                fp32_step("T01", half, "nb1")


(schedule_halves if len(sys.argv) > 1 and sys.argv[1] == "halves" else schedule_steps)()
assert not issued, issued

sys.stdout.write("// generated by gen_gemm2_loop.py (the schedule and its lgkmcnt waits) - edit it there\n" + "\n".join(out) + "\n")
