"""Host-side checks (CPU only): the C ABI library loads and exports every declared symbol, the QPACK2 writer produces
files the reference format readers accept, the synthetic generator is deterministic, and argument errors are reported
through the error channel without touching a GPU."""
import os
import re

import numpy as np
import pytest

import oracle as O
import qpack_amd as qa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    txt = open(os.path.join(ROOT, "include", "qpack_hip.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(qph_[a-z_0-9]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    L = qa.lib()
    syms = declared_symbols()
    assert len(syms) >= 25
    for s in syms:
        assert hasattr(L, s), s
    assert set(syms) == set(qa._lib.SIGNATURES), "ctypes signatures out of sync with include/qpack_hip.h"


def test_device_count_without_gpu_is_not_an_error():
    assert qa.device_count() >= 0


def test_errors_without_gpu():
    with pytest.raises(qa.QphError, match="cannot open"):
        qa.HipLlama.load("/nonexistent/model.qpack")
    q = np.zeros((4, 100), np.int8)
    with pytest.raises(qa.QphError, match="multiple of 128"):
        qa.kernel_matvec(qa.QPH_Q8, q, np.ones(4, np.float32), np.zeros(100, np.float32))


def test_bad_container_is_rejected(tmp_path):
    p = tmp_path / "bad.qpack"
    p.write_bytes(b"NOTQPACK" + b"\0" * 64)
    with pytest.raises(qa.QphError, match="not a QPACK container"):
        qa.HipLlama.load(str(p))
    p.write_bytes(b"QPACK2\0\0" + np.uint32(1).tobytes() + b"\0" * 4 + b"x" * 56 + np.uint64(10 ** 9).tobytes() * 2)
    with pytest.raises(qa.QphError, match="table of contents points outside the file"):
        qa.HipLlama.load(str(p))


@pytest.mark.parametrize("name", ["mini", "mini_q4m"])
def test_synthetic_file_layout(name, tmp_path):
    p = str(tmp_path / "m.qpack")
    qa.write_synthetic(name, p, seed=5)
    f = O.QpackFile(p)
    shape = qa.CONFIGS[name]
    c = f.config
    assert c["arch"] == "llama" and c["hidden_size"] == shape.hidden and c["tie_embeddings"] == shape.tied
    for nm, (off, ln) in f.toc.items():
        assert off % 64 == 0, nm
    # q8 rule (/root/reference/tools/qpack-quantize.cpp:327-339): every row reaches |q| = 127, q in [-127, 127]
    k, q, s, rows, cols = f.tensor("embed")
    assert k == O.OR_Q8 and q.shape == (shape.vocab, shape.hidden)
    assert np.all(np.abs(q.astype(np.int32)).max(1) == 127) and q.min() >= -127
    assert np.all((s > 0.02 * 2 / 127) & (s < 0.02 * 6.5 / 127))   # row absmax of N(0, 0.02) over hundreds of columns
    if shape.q4:
        k, q4, s4, rows, cols = f.tensor("layers.0.wq")
        assert k == O.OR_Q4
        nib = np.concatenate([q4 & 15, q4 >> 4], axis=1)
        assert nib.max() <= 15 and np.any(nib == 1)   # q = -7 present (absmax maps to +-7)
        k2 = f.tensor("layers.0.wv")[0]
        assert k2 == (O.OR_Q8 if shape.q4m_alt else O.OR_Q4)
    n = f.tensor("final_norm")[1]
    assert np.all(n == 1.0)
    f.close()


def test_synthetic_is_deterministic_across_threads(tmp_path):
    a, b, c = (str(tmp_path / f"{i}.qpack") for i in range(3))
    qa.write_synthetic("mini_q4m", a, seed=9, threads=1)
    qa.write_synthetic("mini_q4m", b, seed=9, threads=7)
    qa.write_synthetic("mini_q4m", c, seed=10, threads=7)
    assert open(a, "rb").read() == open(b, "rb").read()
    assert open(a, "rb").read() != open(c, "rb").read()


def test_weights_are_normal(tmp_path):
    p = str(tmp_path / "m.qpack")
    qa.write_synthetic("mini128", p, seed=3, std=0.02)
    f = O.QpackFile(p)
    k, q, s, rows, cols = f.tensor("layers.1.w_up")
    w = q.astype(np.float64) * s[:, None]
    assert abs(w.mean()) < 1e-4 and abs(w.std() - 0.02) < 5e-4
    kurt = ((w - w.mean()) ** 4).mean() / w.var() ** 2
    assert abs(kurt - 3.0) < 0.1
    f.close()


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_reference_reads_synthetic_files(tmp_path):
    p = str(tmp_path / "m.qpack")
    qa.write_synthetic("mini_q4m", p, seed=2)
    r = O.Ref(p, 32)
    assert r.vocab() == qa.CONFIGS["mini_q4m"].vocab and r.hidden() == qa.CONFIGS["mini_q4m"].hidden
    r.close()


REF_QUANT = os.path.join(os.path.dirname(O.REF_LIB), "qpack-quantize")


@pytest.mark.skipif(not os.path.exists(REF_QUANT), reason="oracle/_ref/qpack-quantize not built")
@pytest.mark.parametrize("name,args", [("mini_q1", ["--type", "q1"]), ("mini_q1m", ["--type", "q1m"]),
                                       ("mini_q4mb", ["--type", "q4m"]), ("mini_q4h", ["--type", "q4", "--q4-head"])])
def test_synthetic_policies_match_qpack_quantize(name, args, tmp_path):
    """the synthetic writer puts every tensor in the kind the reference quantiser picks for it (q1 MLP matrices, the q4m
    more_bits layer policy, the q4 head), given the same shape in q8"""
    import dataclasses
    import subprocess
    q8 = dataclasses.replace(qa.CONFIGS[name], q4=False, mlp_q1=False, more_bits=False, q4_head=False)
    src, out, mine = str(tmp_path / "q8.qpack"), str(tmp_path / "ref.qpack"), str(tmp_path / "mine.qpack")
    qa.write_synthetic(q8, src, seed=3)
    subprocess.run([REF_QUANT, src, out] + args, check=True, capture_output=True)
    qa.write_synthetic(name, mine, seed=3)
    kinds = lambda p: {e["name"]: (e["kind"], e.get("group")) for e in O.QpackFile(p).manifest["tensors"]}   # noqa: E731
    assert kinds(mine) == kinds(out)


def _container(path, blobs, magic=b"QPACK2\0\0"):
    """a QPACK container written from Python (16-byte header, 72-byte entries, 64-byte aligned blobs)"""
    n = len(blobs)
    at = (16 + 72 * n + 63) // 64 * 64
    head, body, offs = bytearray(magic + np.uint32(n).tobytes() + b"\0" * 4), bytearray(), []
    for name, data in blobs:
        offs.append(at)
        head += name.encode().ljust(56, b"\0") + np.uint64(at).tobytes() + np.uint64(len(data)).tobytes()
        at = (at + len(data) + 63) // 64 * 64
    out = bytearray(head)
    for (name, data), o in zip(blobs, offs):
        out += b"\0" * (o - len(out)) + data
    open(path, "wb").write(bytes(out))


def test_config_json_reader(tmp_path):
    """the container's JSON reader on hand-written text: whitespace, escapes (\\u0061 -> 'a', a surrogate pair),
    exponents and nesting parse (arch decodes to "llama", so the load reaches the shape checks); malformed text is reported with
    its offset"""
    cfg = (b'{ "arch" : "llam\\u0061", "note": "\\ud83d\\ude00 \\"q\\"\\n", "hidden_size": 8.96e2, "nested": {"a": [1, -2.5e-3, '
           b'true, false, null, {}]}, "num_hidden_layers": 1 }')
    man = b'{"format": "QPACK2", "tensors": []}'
    p = str(tmp_path / "m.qpack")
    _container(p, [("manifest.json", man), ("config.json", cfg)])
    with pytest.raises(qa.QphError, match="bad model config"):
        qa.HipLlama.load(p)
    _container(p, [("manifest.json", man), ("config.json", b'{"arch": "llama", "x": [1, 2,]}')])
    with pytest.raises(qa.QphError, match=r"JSON: .* at offset 29"):
        qa.HipLlama.load(p)
    _container(p, [("manifest.json", man), ("config.json", b'{"arch": "lfm2"}')])
    with pytest.raises(qa.QphError, match="not a Llama-family model"):
        qa.HipLlama.load(p)


def test_bench_graph_timeline_summary(tmp_path):
    """bench.py's graph_timeline(): per-kernel mean in-kernel time (first start to last end, 100 MHz ticks -> us), the
    mean gap between consecutive launches by kernel pair, and the share of the span inside launches."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("bench", os.path.join(os.path.dirname(__file__), "..", "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    # two layers and the head: qkv 0-700, attn 800-1700, gate_up 1850-3800, down 3950-5200, then again, head
    rows, t = [], 0
    for _ in range(2):
        for name, dur, gap in (("qkv", 700, 100), ("attn_wo", 900, 150), ("gate_up", 1950, 150), ("down", 1250, 150)):
            rows.append((name, t, t + dur)); t += dur + gap
    rows.append(("head", t, t + 8000))
    p = tmp_path / "tl.txt"
    p.write_text("".join(f"{n} {a} {b}\n" for n, a, b in rows))
    s = bench.graph_timeline(str(p))
    assert s["launches"] == 9
    assert s["kernel_mean_us"] == {"qkv": 7.0, "attn_wo": 9.0, "gate_up": 19.5, "down": 12.5, "head": 80.0}
    assert s["gap_mean_us"] == {"qkv->attn_wo": 1.0, "attn_wo->gate_up": 1.5, "gate_up->down": 1.5,
                                "down->qkv": 1.5, "down->head": 1.5}
    span = (rows[-1][2] - rows[0][1]) / 100.0
    busy = sum(b - a for _, a, b in rows) / 100.0
    assert s["span_us"] == round(span, 1) and s["kernel_us"] == round(busy, 1)
    assert s["kernel_frac"] == round(busy / span, 4)
