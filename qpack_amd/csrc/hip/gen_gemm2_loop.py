"""Writes gemm2_loop.inc: the per-block body of k_gemm2_q8's main loop (prefill.hip), a fixed schedule of LDS fragment
reads, int8 MFMAs and VALU steps, and (the G2_TAIL section) the fp32 steps the loop leaves for after its last block.

The LDS reads are inline asm (the compiler cannot see which direct-to-LDS load fills which stage), so every use of a
read's result must follow an explicit `s_waitcnt lgkmcnt(N)` naming it.  N depends on how many reads were issued after
it; this script tracks the issue order and computes each N, so an edit of the schedule cannot leave a wrong count.
Run it after editing:  python3 gen_gemm2_loop.py > gemm2_loop.inc   (argument: a schedule name, default "pairs")

One 128-column block: K = 4 steps of 32; the wave's 64 x 64 tile is rows mi0 / mi1 x tokens ni0 / ni1, one int32
accumulator T[mi][ni] each.  Per tile and block: 4 hi-plane MFMAs, the shift-add T = 256 T + 128 sum(W) (16 VALU), 4
lo-plane MFMAs, the fp32 step acc = fma(bs, (float) T, acc) (32 VALU).  Measured on the 28672 x 4096 x 2048 product:
the VALU work and the LDS reads each co-issue with the MFMAs alone (~280 us with either removed), but together they
contend (the LDS results and the VALU results share the register-file writes), so the schedules differ in how evenly
the VALU work is spread over the MFMAs and in how many fragment bytes each block reads:
  steps    4 MFMAs (all four tiles) per 32-deep step, 34 reads; VALU in three bursts           573 us
  halves   quarters of 8 MFMAs on one row half, 50 reads                                        (= steps)
  eighths  groups of 4 MFMAs on one tile, ~6 VALU per MFMA, 48 reads                             554 us
  pairs    eighths in the order T00 T10 T01 T11: consecutive groups share token fragments, 34 reads  512 us
"""
import sys

LOOK = 2

out = []
issued = []   # LDS reads in flight, oldest first


def emit(s):
    out.append("    " + s)


def read(name, expr):
    if len(issued) == 15:   # the 4-bit lgkmcnt: land the oldest first
        wait(issued[0])
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


def schedule_eighths():
    """Eight groups of 4 MFMAs, one tile and one plane each: E1..E4 the hi plane of T00, T01, T10, T11, E5..E8 the lo
    plane in the same order.  Each tile's VALU work - its shift-add S (16 instructions) after its hi group and before
    its lo group, its fp32 step F (32) after its lo group and before the next block's hi group of the same tile - is cut
    into units of 8 instructions and dealt 3 units to every group, so each MFMA has ~6 VALU instructions of other tiles
    beside it:
        E1 F10 F10 F10 | E2 F10 F11 S00 | E3 F11 F11 F11 | E4 S00 S01 S10
        E5 S01 S10 S11 | E6 S11 F00 F00 | E7 F00 F00 F01 | E8 F01 F01 F01
    (F10 / F11 take the previous block's token scales, F00 / F01 this block's).  A unit whose tile's MFMAs have just
    ended comes last in its group.  `__builtin_amdgcn_sched_barrier(0)` after each MFMA and its VALU share keeps the
    compiler from regrouping them.  Token fragments roll through one register set: the read for group g + 1, step ks
    is issued right after group g's MFMA of step ks (4 MFMAs of cover).  A fragments are read with the hi group of
    their row half's first tile and held for its lo groups."""
    groups = [("h", 0, 0), ("h", 0, 1), ("h", 1, 0), ("h", 1, 1), ("l", 0, 0), ("l", 0, 1), ("l", 1, 0), ("l", 1, 1)]
    units = [["F10", "F10", "F10"], ["F10", "F11", "S00"], ["F11", "F11", "F11"], ["S00", "S01", "S10"],
             ["S01", "S10", "S11"], ["S11", "F00", "F00"], ["F00", "F00", "F01"], ["F01", "F01", "F01"]]
    dealt = {}   # elements of each tile's S / F already dealt

    def unit_ops(u):
        """the next 8 VALU instructions of unit u: (C statement, instructions, LDS-read registers it needs)"""
        kind, mi, ni = u[0], int(u[1]), int(u[2])
        k = dealt.get(u, 0)
        ops = []
        if kind == "S":
            w = "w" if mi == 0 else "x"
            for i in range(k, k + 8):
                ops.append((f"T[{mi}][{ni}][{i}] = T[{mi}][{ni}][{i}] * 256 + {w}{i // 4}[{i % 4}];", 1, [f"{w}{i // 4}"]))
            dealt[u] = k + 8
        else:
            bs = ("pb" if mi == 1 else "nb") + str(ni)
            for i in range(k, k + 4):
                ops.append((f"acc[{mi}][{ni}][{i}] = __builtin_fmaf({bs}, (float)T[{mi}][{ni}][{i}], acc[{mi}][{ni}][{i}]);",
                            2, [bs] if mi == 0 else []))
            dealt[u] = k + 4
        return ops

    def read_frag(g, ks):
        plane, mi, ni = groups[g]
        if plane == "h" and ni == 0:
            read(f"A{mi}[{ks}]", RA(ks, mi))
        read(f"bq[{ks}]", RB(plane, ks, ni))

    def need(*regs):
        pend = [r for r in regs if r in issued]
        if pend:
            wait(*pend)

    for ks in range(4):
        read_frag(0, ks)
    extras_ws(0, "w")()          # S00 from the end of E2
    for g, (plane, mi, ni) in enumerate(groups):
        emit(f"// ---- E{g + 1}: {'hi' if plane == 'h' else 'lo'} plane of T{mi}{ni} || {' '.join(units[g])}")
        ops = [op for u in units[g] for op in unit_ops(u)]
        total = sum(o[1] for o in ops)
        shares, run = [[] for _ in range(4)], 0
        for op in ops:   # by instruction count: ~total / 4 after each MFMA
            shares[min(3, (4 * run) // total)].append(op)
            run += op[1]
        for ks in range(4):
            need(f"A{mi}[{ks}]", f"bq[{ks}]")
            t = f"T[{mi}][{ni}]"
            first = plane == "h" and ks == 0
            emit(f"{t} = __builtin_amdgcn_mfma_i32_32x32x32_i8(A{mi}[{ks}], bq[{ks}], {'zero' if first else t}, 0, 0, 0);")
            if g + 1 < len(groups):
                read_frag(g + 1, ks)
            if ks == 0 and g == 2:
                extras_ws(1, "x")()  # S10 at the end of E4
            if ks == 0 and g == 4:
                extras_bs()          # F00 from E6
            for stmt, _, regs in shares[ks]:
                need(*regs)
                emit(stmt)
            emit("__builtin_amdgcn_sched_barrier(0);")
    for u, n in dealt.items():
        assert n == 16, (u, n)


def schedule_pairs():
    """The eighths' VALU dealing with the tiles taken in the order T00, T10, T01, T11 (hi plane: groups E1..E4; lo
    plane: E5..E8), so consecutive groups share their token fragments: one rolling set is read for each pair of groups
    (E1 E2: hi plane of tokens ni0, E3 E4: ni1, then the lo plane likewise), 34 LDS reads per block instead of 48.
    Units by position p0..p3 = T00, T10, T01, T11:
        E1 F2 F2 F2 | E2 F2 F3 S0 | E3 F3 F3 F3 | E4 S0 S1 S2
        E5 S1 S2 S3 | E6 S3 F0 F0 | E7 F0 F0 F1 | E8 F1 F1 F1
    F0 / F1 take this block's token scale, F2 / F3 (T01, T11: run under the next block's first groups) the previous
    block's.  After the loop the last block's F2 / F3 are still due: the G2_TAIL section of this file."""
    pos = [(0, 0), (1, 0), (0, 1), (1, 1)]
    groups = [("h", p) for p in range(4)] + [("l", p) for p in range(4)]
    units = [["F2", "F2", "F2"], ["F2", "F3", "S0"], ["F3", "F3", "F3"], ["S0", "S1", "S2"],
             ["S1", "S2", "S3"], ["S3", "F0", "F0"], ["F0", "F0", "F1"], ["F1", "F1", "F1"]]
    dealt = {}

    def fstmt(p, i, bs):
        mi, ni = pos[p]
        return f"acc[{mi}][{ni}][{i}] = __builtin_fmaf({bs}, (float)T[{mi}][{ni}][{i}], acc[{mi}][{ni}][{i}]);"

    def scale(p):
        return ("nb" if p < 2 else "pb") + str(pos[p][1])

    def unit_ops(u):
        kind, p = u[0], int(u[1])
        mi, ni = pos[p]
        k = dealt.get(u, 0)
        ops = []
        if kind == "S":
            w = "w" if mi == 0 else "x"
            for i in range(k, k + 8):
                ops.append((f"T[{mi}][{ni}][{i}] = T[{mi}][{ni}][{i}] * 256 + {w}{i // 4}[{i % 4}];", 1, [f"{w}{i // 4}"]))
            dealt[u] = k + 8
        else:
            bs = scale(p)
            for i in range(k, k + 4):
                ops.append((fstmt(p, i, bs), 2, [bs] if p < 2 else []))
            dealt[u] = k + 4
        return ops

    def need(*regs):
        pend = [r for r in regs if r in issued]
        if pend:
            wait(*pend)

    for ks in range(4):
        read(f"A0[{ks}]", RA(ks, 0))
        read(f"bq[{ks}]", RB("h", ks, 0))
    extras_ws(0, "w")()          # S0 from the end of E2
    for g, (plane, p) in enumerate(groups):
        mi, ni = pos[p]
        emit(f"// ---- E{g + 1}: {'hi' if plane == 'h' else 'lo'} plane of T{mi}{ni} || {' '.join(units[g])}")
        ops = [op for u in units[g] for op in unit_ops(u)]
        total = sum(o[1] for o in ops)
        shares, run = [[] for _ in range(4)], 0
        for op in ops:
            shares[min(3, (4 * run) // total)].append(op)
            run += op[1]
        for ks in range(4):
            need(f"A{mi}[{ks}]", f"bq[{ks}]")
            t = f"T[{mi}][{ni}]"
            first = plane == "h" and ks == 0
            emit(f"{t} = __builtin_amdgcn_mfma_i32_32x32x32_i8(A{mi}[{ks}], bq[{ks}], {'zero' if first else t}, 0, 0, 0);")
            if g == 0:
                read(f"A1[{ks}]", RA(ks, 1))     # for E2
            if g % 2 == 1 and g + 1 < len(groups):
                nplane, np_ = groups[g + 1]
                read(f"bq[{ks}]", RB(nplane, ks, pos[np_][1]))
            if ks == 0 and g == 2:
                extras_ws(1, "x")()  # S1 (T10) from E4
            if ks == 0 and g == 4:
                extras_bs()          # F0 from E6
            for stmt, _, regs in shares[ks]:
                need(*regs)
                emit(stmt)
            emit("__builtin_amdgcn_sched_barrier(0);")
    for u, n in dealt.items():
        assert n == 16, (u, n)
    # after the loop: the last block's fp32 steps of positions 2 and 3
    out.append("#else")
    for p in (2, 3):
        for i in range(16):
            emit(fstmt(p, i, scale(p)))


SCHEDULES = {"steps": schedule_steps, "halves": schedule_halves, "eighths": schedule_eighths, "pairs": schedule_pairs}
out.append("#ifndef G2_TAIL")
name = sys.argv[1] if len(sys.argv) > 1 else "pairs"
SCHEDULES[name]()
if name != "pairs":   # the other schedules defer the fp32 steps of rows mi1
    out.append("#else")
    for mi_ni in ("1][0", "1][1"):
        for i in range(16):
            emit(f"acc[{mi_ni}][{i}] = __builtin_fmaf(pb{mi_ni[-1]}, (float)T[{mi_ni}][{i}], acc[{mi_ni}][{i}]);")
out.append("#endif")
assert not issued, issued

sys.stdout.write("// generated by gen_gemm2_loop.py (the schedule and its lgkmcnt waits) - edit it there\n" + "\n".join(out) + "\n")
