"""QPACK3 rANS on the CPU: the oracle codec against the reference's own blobs (tests/golden/rans.npz) and against the
reference codec compiled from its sources (oracle/_ref), the encoder's frequency invariants, and the product's packer
(qph_pack, host code) against the reference qpack-pack and the oracle's restatement of it.  The GPU decoder's tests are
in test_gpu_rans.py."""
import json
import os
import subprocess

import numpy as np
import pytest

import oracle as O
import qpack_amd as qa

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "rans.npz")
REF_PACK = os.path.join(os.path.dirname(O.REF_LIB), "qpack-pack")


def golden():
    z = np.load(GOLDEN)
    cases = [(int(i), int(c), int(p), z[f"raw{i}"], z[f"blob{i}"]) for i, c, p, _ in z["meta"]]
    errors = dict(s.split("\t") for s in z["errors"])
    return cases, {k: z[f"bad_{k}"] for k in errors}, errors


def test_oracle_matches_reference_blobs():
    cases, _, _ = golden()
    assert len(cases) >= 80
    for i, codec, planes, raw, blob in cases:
        assert np.array_equal(O.rans_encode(raw, codec, planes), blob), f"case {i}: encoder differs"
        assert np.array_equal(O.rans_decode(blob), raw), f"case {i}: decoder differs"


def test_oracle_errors_match_reference():
    _, bad, errors = golden()
    for k, b in bad.items():
        with pytest.raises(ValueError) as e:
            O.rans_decode(b)
        assert str(e.value) == errors[k], (k, e.value)


def test_frequency_table_invariants():
    """sum 4096 and a frequency exactly for the symbols that occur; the floors max(1, h * 4096 // n) are kept except for
    the most frequent symbol (first on ties), which takes the rest - or, where the floors already exceed 4096, they
    only shrink (the largest first) and none drops below 1"""
    rng = np.random.default_rng(7)
    L = O.olib()
    for n, nsym, kind in [(1, 256, "u"), (10, 256, "u"), (300, 256, "u"), (5000, 256, "u"), (100000, 256, "g"),
                          (999, 16, "u"), (50000, 16, "g"), (4097, 256, "u")]:
        s = rng.integers(0, nsym, n).astype(np.uint8) if kind == "u" else np.clip(rng.normal(nsym / 2, 2, n), 0, nsym - 1).astype(np.uint8)
        f = np.zeros(256, np.uint32)
        assert L.or_rans_freqs(O._p(s), n, nsym, O._p(f)) == 0
        f = f[:nsym].astype(np.int64)
        h = np.bincount(s, minlength=nsym)[:nsym]
        assert f.sum() == 4096 and np.array_equal(f > 0, h > 0)
        fl = np.where(h > 0, np.maximum(h * 4096 // n, 1), 0)
        big = int(np.argmax(h))
        rest = 4096 - fl.sum() + fl[big]
        if rest >= 1:
            expect = fl.copy(); expect[big] = rest
            assert np.array_equal(f, expect)
        else:
            assert (f <= fl).all() and f[h > 0].min() >= 1


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built")
def test_oracle_matches_live_reference_codec():
    import ctypes as C
    L = O.rlib(1)
    rng = np.random.default_rng(11)
    for n in [0, 1, 7, 513, 4096, 30001]:
        for codec, planes in [(1, 1), (1, 2), (1, 4), (2, 1)]:
            for raw in (rng.integers(0, 256, n, dtype=np.uint8), np.clip(rng.normal(100, 1.5, n), 0, 255).astype(np.uint8)):
                cap = 4 * n + 4096
                out = np.empty(cap, np.uint8)
                m = C.c_int64()
                assert L.qpref_rans_encode(O._p(raw), n, codec, planes, O._p(out), cap, C.byref(m)) == 0
                assert np.array_equal(O.rans_encode(raw, codec, planes), out[:m.value])
                dec = np.zeros(n + 16, np.uint8)
                assert L.qpref_rans_decode(O._p(out), m.value, O._p(dec)) == 0
                assert np.array_equal(dec[:n], raw)


def test_chunked_blob_round_trip():
    rng = np.random.default_rng(3)
    raw = np.clip(rng.normal(128, 5, 10000), 0, 255).astype(np.uint8)
    chunks = [O.rans_encode(raw[o:o + 4096], 1, 1) for o in range(0, len(raw), 4096)]
    blob = O.rans_assemble_chunked(len(raw), 4096, chunks)
    assert O.rans_raw_size(blob) == len(raw)
    assert np.array_equal(O.rans_decode(blob), raw)


def same_files(a_path, b_path):
    a, b = O.QpackFile(a_path), O.QpackFile(b_path)
    order = lambda f: sorted(f.toc, key=lambda n: f.toc[n][0])   # noqa: E731
    assert order(a) == order(b)
    for n in a.toc:
        ra = bytes(a.mm[a.toc[n][0]:a.toc[n][0] + a.toc[n][1]])
        rb = bytes(b.mm[b.toc[n][0]:b.toc[n][0] + b.toc[n][1]])
        if n == "manifest.json":   # the reference's JSON writer prints floats with fewer digits
            ja, jb = json.loads(ra), json.loads(rb)
            assert all(ja[k] == jb[k] for k in ("format", "tensors", "encoded")), n
        else:
            assert ra == rb, n
    return a, b


@pytest.mark.parametrize("name", ["mini", "mini_q4m"])
def test_product_packer_matches_oracle_packer(name, tmp_path):
    src = str(tmp_path / "m.qpack")
    qa.write_synthetic(name, src, seed=9)
    n = qa.pack(src, str(tmp_path / "p.qpack"), 4)
    enc = O.pack_qpack3(src, str(tmp_path / "o.qpack"))
    assert n == len(enc) > 0
    a, _ = same_files(str(tmp_path / "p.qpack"), str(tmp_path / "o.qpack"))
    assert a.mm[:8] == b"QPACK3\0\0" and a.manifest["format"] == "QPACK3"
    # the coded file reads back to the source's tensors
    s = O.QpackFile(src)
    for t in s.tensors:
        for x, y in zip(s.tensor(t)[1:3], a.tensor(t)[1:3]):
            assert (x is None and y is None) or np.array_equal(x, y), t


@pytest.mark.skipif(not os.path.exists(REF_PACK), reason="oracle/_ref/qpack-pack not built")
@pytest.mark.parametrize("name", ["mini", "mini_q4"])
def test_product_packer_matches_reference_qpack_pack(name, tmp_path):
    src = str(tmp_path / "m.qpack")
    qa.write_synthetic(name, src, seed=4)
    qa.pack(src, str(tmp_path / "p.qpack"), 3)
    subprocess.run([REF_PACK, src, str(tmp_path / "r.qpack"), "-t", "2"], check=True, capture_output=True)
    same_files(str(tmp_path / "p.qpack"), str(tmp_path / "r.qpack"))


def test_packer_rejects_non_qpack2(tmp_path):
    src = str(tmp_path / "m.qpack")
    qa.write_synthetic("mini", src, seed=1)
    qa.pack(src, str(tmp_path / "p.qpack"), 2)
    with pytest.raises(qa.QphError, match="needs a QPACK2 file"):
        qa.pack(str(tmp_path / "p.qpack"), str(tmp_path / "q.qpack"), 2)
