"""The reference-side binding, compiled: the qp::Model adapter (qpack_amd/integration/model_llama_hip.cpp) built against
the reference's own headers (/root/reference/include/qpack/qpack.h:128-177) and sources, and linked with
libqpack_hip.so into the reference's qpack-bench (tools/qpack-bench.cpp) with the QPACK_DEVICE=hip branch of
load_model (model_llama.cpp:221-235).  On the CPU the binary must run the reference engine unchanged and report the
missing GPU through the adapter's error path; on a GPU box (-m gpu) it runs a C1 row on the HIP model.

adapter_check (qpack_amd/integration/adapter_check.cpp) links the same objects and checks what the adapter computes:
the C1 greedy stream through load_model / prefill / greedy_run against the reference's own (tests/golden/c1.json), and
the device-sampler glue (sampler_hip.cpp): Sampler::dist from the device top-M equal bit for bit to Sampler::dist on
the full logits (/root/reference/src/sampler.cpp:12-57), and the same token drawn."""
import json
import os
import subprocess

import pytest

import qpack_amd as qa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "qpack_amd", "integration", "_build", "qpack-bench")
CHECK = os.path.join(ROOT, "qpack_amd", "integration", "_build", "adapter_check")
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


def check(args, device="hip", order=None, timeout=600):
    env = dict(os.environ)
    env.pop("QPACK_DEVICE", None)
    env.pop("QPACK_HIP_ORDER", None)
    if device:
        env["QPACK_DEVICE"] = device
    if order:
        env["QPACK_HIP_ORDER"] = order
    return subprocess.run([CHECK] + [str(a) for a in args], env=env, capture_output=True, text=True, timeout=timeout)


@pytest.mark.skipif(not os.path.exists(CHECK), reason="adapter_check is built where the reference is")
def test_candidate_dist_equals_reference_dist_cpu():
    """dist_from_candidates on the exact top-M (a host full sort) against the reference's Sampler::dist on the full
    logits: 151936 random logits with ties at the top and signed zeros; top_k 1 / 40 / 448 / 512, repeat penalty 1 /
    1.1 / 0.9, temperature 0 / 0.7 / 1.3, top-p and min-p on and off; distributions bit-identical, draws equal"""
    r = check(["candidates-cpu", 7], device=None)
    print(r.stdout[-400:], r.stderr[-400:])
    assert r.returncode == 0, r.stdout + r.stderr
    assert "different 0" in r.stdout


@pytest.mark.skipif(not os.path.exists(CHECK), reason="adapter_check is built where the reference is")
def test_adapter_reference_engine_greedy_cpu(tmp_path):
    """the harness itself against the reference engine (no QPACK_DEVICE): prefill + greedy_run on a small model equal
    to the oracle's stream, so the GPU leg below compares like with like"""
    import oracle
    import numpy as np
    p = str(tmp_path / "mini.qpack")
    qa.write_synthetic("mini", p, seed=3)
    toks = [5, 77, 300, 12, 9, 100, 41, 2]
    r = check(["greedy", p, 12] + toks, device=None)
    assert r.returncode == 0, r.stderr
    lines = dict(l.split(" ", 1) for l in r.stdout.strip().splitlines())
    o = oracle.Oracle(p, max_ctx=40)
    lg = o.prefill(np.array(toks, np.int32), 1)
    first = int(np.argmax(lg))
    want = o.greedy_run(first, 12)
    o.close()
    assert int(lines["first"]) == first
    assert [int(t) for t in lines["greedy"].split()] == want.tolist()
    assert lines["arch"] == "llama:qwen2"


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
    assert cells[2] == "llama:qwen2@hip"   # the backend's mark, like the CUDA model's "@cuda"
    pp, tg = float(cells[4]), float(cells[5])
    assert pp > 100 and tg > 100   # the CPU engine does ~10-40 tok/s here; the HIP model runs hundreds


def c1_fixture():
    with open(os.path.join(ROOT, "tests", "golden", "c1.json")) as f:
        return json.load(f)


@pytest.mark.gpu
@pytest.mark.skipif(not os.path.exists(CHECK), reason="adapter_check is built where the reference is")
def test_adapter_greedy_equals_reference(synth):
    """C1 through the adapter as a reference caller drives it (load_model with QPACK_DEVICE=hip, prefill, greedy_run,
    container()): in the reference order the first token and all 128 greedy tokens equal the reference's stream; in
    the default order the stream agrees up to the reference's first near-tie (top-2 gap 4e-5 at step 61)"""
    fx = c1_fixture()
    path = synth("c1")
    n = len(fx["greedy"])
    for order in ("reference", "default"):
        r = check(["greedy", path, n] + fx["prompt"], order=order)
        print(order, r.stdout[:300], r.stderr[-300:], flush=True)
        assert r.returncode == 0, r.stderr
        lines = dict(l.split(" ", 1) for l in r.stdout.strip().splitlines())
        assert lines["arch"] == "llama:qwen2@hip"
        assert int(lines["file_size"]) == os.path.getsize(path)
        assert int(lines["first"]) == fx["first_token"]
        got = [int(t) for t in lines["greedy"].split()]
        if order == "reference":
            assert got == fx["greedy"], "the adapter's greedy stream differs from the reference's"
        else:
            agree = next((i for i, (a, b) in enumerate(zip(got, fx["greedy"])) if a != b), n)
            assert agree >= 61, f"default order: greedy agrees for {agree}/{n} tokens only"


@pytest.mark.gpu
@pytest.mark.skipif(not os.path.exists(CHECK), reason="adapter_check is built where the reference is")
@pytest.mark.parametrize("top_k,penalty,temp", [(1, 1.1, 0.7), (40, 1.1, 0.7), (40, 1.0, 1.3), (448, 1.1, 1.0),
                                                (512, 1.0, 0.7), (512, 1.1, 0.7), (40, 1.1, 0.0)])
def test_device_candidates_sample_like_the_logits(synth, top_k, penalty, temp):
    """Session's sampling on the HIP model (C1, 24 steps after the C1 prompt): Sampler::dist on step(tok, 1)'s logits,
    dist_from_candidates on qph_step_topk's M = top_k + |penalised| candidates, and hip_sample_step give bit-identical
    distributions and draw the same tokens from samplers of one seed.  top_k 512 with penalties needs more than the
    device's 512 candidates, so hip_sample_step takes the logits there (device_steps 0)"""
    fx = c1_fixture()
    path = synth("c1")
    r = check(["sample", path, 24, top_k, penalty, temp, 1234] + fx["prompt"])
    print(r.stdout[-600:], r.stderr[-300:], flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    tail = r.stdout.strip().splitlines()[-1].split()
    device_steps = int(tail[1])
    assert tail[3] == "0"
    if top_k + (1 if penalty != 1.0 else 0) <= 512 and not (top_k == 512 and penalty != 1.0):
        assert device_steps == 24
    else:
        assert device_steps == 0
