"""The reference-side binding, compiled: the qp::Model adapter (qpack_amd/integration/model_llama_hip.cpp) built against
the reference's own headers (/root/reference/include/qpack/qpack.h:128-177) and sources, and linked with
libqpack_hip.so into the reference's qpack-bench (tools/qpack-bench.cpp) with the QPACK_DEVICE=hip branch of
load_model (model_llama.cpp:221-235).  On the CPU the binary must run the reference engine unchanged and report the
missing GPU through the adapter's error path; on a GPU box (-m gpu) it runs a C1 row on the HIP model."""
import os
import subprocess

import pytest

import qpack_amd as qa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "qpack_amd", "integration", "_build", "qpack-bench")
REF = "/root/reference"


def row(path, device, extra=()):
    env = dict(os.environ)
    env.pop("QPACK_DEVICE", None)
    if device:
        env["QPACK_DEVICE"] = device
    return subprocess.run([BENCH, "--row", "-m", path, "-t", "4", "-r", "1"] + list(extra), env=env, capture_output=True,
                          text=True, timeout=600)


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src")), reason="the reference sources are not here")
def test_adapter_builds_and_links(tmp_path):
    subprocess.run(["make", "-C", os.path.join(ROOT, "qpack_amd", "integration"), "REF=" + REF, "-j8"], check=True,
                   capture_output=True)
    assert os.path.exists(BENCH)
    p = str(tmp_path / "mini.qpack")
    qa.write_synthetic("mini", p, seed=3)
    r = row(p, None, ["-p", "8", "-n", "4"])   # the reference CPU engine through the same binary
    assert r.returncode == 0, r.stderr
    cells = [c.strip() for c in r.stdout.strip().strip("|").split("|")]
    assert cells[0] == "mini.qpack" and cells[2].startswith("llama") and float(cells[5]) > 0
    if qa.device_count() == 0:   # the HIP branch is taken and reports that no device is there
        r = row(p, "hip", ["-p", "8", "-n", "4"])
        assert r.returncode != 0 and "hip:" in r.stderr


@pytest.mark.gpu
@pytest.mark.skipif(not os.path.exists(BENCH), reason="qpack-bench with the HIP adapter is built where the reference is")
def test_reference_bench_runs_the_hip_model(synth):
    """QPACK_DEVICE=hip qpack-bench --row -m c1.qpack -p 32 -n 128 --greedy: the reference's own benchmark driver on
    the HIP model through the adapter"""
    path = synth("c1")
    r = row(path, "hip", ["-p", "32", "-n", "128", "--greedy"])
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    cells = [c.strip() for c in r.stdout.strip().strip("|").split("|")]
    assert cells[2] == "llama:qwen2"
    pp, tg = float(cells[4]), float(cells[5])
    assert pp > 100 and tg > 100   # the CPU engine does ~10-40 tok/s here; the HIP model runs hundreds
