"""The generated block schedule of the 32 x 32 q8 prompt product (qpack_amd/csrc/hip/gemm2_loop.inc, written by
gen_gemm2_loop.py): the committed file is the generator's current output, and, read back as text, every value an LDS
read delivers is waited for (an `s_waitcnt lgkmcnt(N)` naming it, N = the reads issued after it) before any use, with
at most 15 reads in flight (the 4-bit lgkmcnt).  The reads are inline asm, so the compiler cannot check these waits."""
import os
import re
import subprocess
import sys

HIP = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "qpack_amd", "csrc", "hip")


def generate(*args):
    return subprocess.run([sys.executable, os.path.join(HIP, "gen_gemm2_loop.py"), *args], check=True,
                          capture_output=True, text=True).stdout


def test_committed_schedule_is_the_generators_output():
    with open(os.path.join(HIP, "gemm2_loop.inc")) as f:
        assert f.read() == generate(), "gemm2_loop.inc is stale: run gen_gemm2_loop.py > gemm2_loop.inc"


READ = re.compile(r"^\s*(\S+) = lds_read(?:16|4)o<")
WAIT = re.compile(r'^\s*asm volatile\("s_waitcnt lgkmcnt\((\d+)\)" : (.*)\);')
OPND = re.compile(r'"\+v"\(([^)]+)\)')


def check_schedule(text):
    inflight, landed = [], set()
    for line in text.splitlines():
        m = READ.match(line)
        if m:
            reg = m.group(1)
            landed.discard(reg)
            inflight.append(reg)
            assert len(inflight) <= 15, f"more than 15 LDS reads in flight at: {line.strip()}"
            continue
        m = WAIT.match(line)
        if m:
            n = int(m.group(1))
            done, inflight = inflight[:len(inflight) - n], inflight[len(inflight) - n:]
            named = set(OPND.findall(m.group(2)))
            assert named == set(done), f"wait names {sorted(named)}, lands {sorted(done)}"
            landed |= named
            continue
        # any other statement: the registers it uses must have landed
        for reg in set(inflight):
            if re.search(r"(?<![\w\]])" + re.escape(reg) + r"(?![\w\[])", line):
                raise AssertionError(f"{reg} used before its read landed: {line.strip()}")
    assert not inflight, f"reads still in flight at the end of the block: {inflight}"


def test_schedule_waits_cover_every_use():
    for name in ("pairs", "eighths", "steps", "halves"):
        check_schedule(generate(name))


def test_checker_catches_a_missing_wait():
    text = generate()
    lines = text.splitlines()
    i = next(k for k, l in enumerate(lines) if WAIT.match(l))
    broken = "\n".join(lines[:i] + lines[i + 1:])
    try:
        check_schedule(broken)
    except AssertionError:
        return
    raise AssertionError("a schedule without its first wait passed the check")
