"""QPACK3 rANS decode on the GPU (qph_kernel_rans_decode, and qph_load of a QPACK3 file) against the reference codec:
the reference's own blobs and error messages (tests/golden/rans.npz), the oracle's decoder on seeded blobs of every
codec / plane count / statistics, chunked blobs (including chunk sizes that are not multiples of 8, which take the
byte-store path), and a model whose QPACK3 file must give exactly the logits of its QPACK2 file.  Bit-exact throughout."""
import numpy as np
import pytest

import oracle as O
import qpack_amd as qa

from test_rans import golden

pytestmark = pytest.mark.gpu


def gpu_decode(blob):
    out, ms = qa.kernel_rans_decode(np.ascontiguousarray(blob, np.uint8))
    return out


def test_reference_blobs():
    cases, _, _ = golden()
    for i, codec, planes, raw, blob in cases:
        print(f"rans golden case {i} codec {codec} planes {planes} n {len(raw)}", flush=True)
        np.testing.assert_array_equal(gpu_decode(blob), raw, err_msg=f"case {i}")


def test_reference_error_messages():
    _, bad, errors = golden()
    for k, b in bad.items():
        print(f"rans error case {k}", flush=True)
        with pytest.raises(qa.QphError) as e:
            gpu_decode(b)
        assert errors[k] in str(e.value), (k, str(e.value), errors[k])


def raw_of(rng, kind, n):
    if kind == "uniform":
        return rng.integers(0, 256, n, dtype=np.uint8)
    if kind == "narrow":
        return np.clip(rng.normal(128, 2.5, n), 0, 255).astype(np.uint8)
    if kind == "zeros":
        return np.zeros(n, np.uint8)
    return np.where(rng.random(n) < 0.9995, 3, 250).astype(np.uint8)   # one symbol near probability 1


@pytest.mark.parametrize("kind", ["uniform", "narrow", "zeros", "skewed"])
@pytest.mark.parametrize("codec,planes", [(1, 1), (1, 2), (1, 3), (1, 4), (2, 1)])
def test_random_blobs(kind, codec, planes):
    rng = np.random.default_rng(hash((kind, codec, planes)) % 2 ** 32)
    for n in [1, 4, 7, 8, 255, 256, 257, 511, 512, 513, 2048, 4099, 70001]:
        raw = raw_of(rng, kind, n)
        blob = O.rans_encode(raw, codec, planes)
        print(f"rans random {kind} codec {codec} planes {planes} n {n}", flush=True)
        np.testing.assert_array_equal(gpu_decode(blob), O.rans_decode(blob))
        np.testing.assert_array_equal(gpu_decode(blob), raw)


@pytest.mark.parametrize("chunk", [1000, 4096, 65536])
@pytest.mark.parametrize("codec", [1, 2])
def test_chunked_blobs(chunk, codec):
    rng = np.random.default_rng(chunk + codec)
    raw = np.clip(rng.normal(100, 4, 300000), 0, 255).astype(np.uint8)
    chunks = [O.rans_encode(raw[o:o + chunk], codec, 1) for o in range(0, len(raw), chunk)]
    blob = O.rans_assemble_chunked(len(raw), chunk, chunks)
    print(f"rans chunked chunk {chunk} codec {codec}", flush=True)
    np.testing.assert_array_equal(gpu_decode(blob), raw)


@pytest.mark.parametrize("round_bytes", [0, 520, 600, 1037, 4096, 65536])
def test_streamed_rounds(round_bytes, monkeypatch):
    """the upload in rounds of round_bytes per plane (QPH_RANS_ROUND), each followed by a decode launch that takes every
    plane as far as its uploaded bytes allow: planes stop between steps, keep their states and resume in the next launch.
    Bit-exact for every round size, with planes of unequal length (a chunked blob with a short last chunk and a two-plane
    codec-1 blob), and an overrun still reported"""
    monkeypatch.setenv("QPH_RANS_ROUND", str(round_bytes))
    rng = np.random.default_rng(round_bytes + 11)
    raw = np.clip(rng.normal(100, 6, 150000), 0, 255).astype(np.uint8)
    C = 40000
    blob = O.rans_assemble_chunked(len(raw), C, [O.rans_encode(raw[o:o + C], 1, 1) for o in range(0, len(raw), C)])
    print(f"rans streamed rounds {round_bytes}: chunked", flush=True)
    np.testing.assert_array_equal(gpu_decode(blob), raw)
    raw2 = raw_of(rng, "uniform", 30001)
    print(f"rans streamed rounds {round_bytes}: codec 1 planes 2", flush=True)
    np.testing.assert_array_equal(gpu_decode(O.rans_encode(raw2, 1, 2)), raw2)
    b = O.rans_encode(raw2, 1, 1)
    cl = int(np.frombuffer(b[6:10].tobytes(), np.uint32)[0])
    b[6:10] = np.frombuffer(np.uint32(cl - 3000).tobytes(), np.uint8)
    print(f"rans streamed rounds {round_bytes}: overrun", flush=True)
    with pytest.raises(qa.QphError, match="stream overrun"):
        gpu_decode(b)


def test_overrun_matches_oracle():
    rng = np.random.default_rng(5)
    blob = O.rans_encode(rng.integers(0, 256, 5000, dtype=np.uint8), 1, 1)
    cl = int(np.frombuffer(blob[6:10].tobytes(), np.uint32)[0])
    for cut in [1, 7, 100, 4000]:
        b = blob.copy()
        b[6:10] = np.frombuffer(np.uint32(cl - cut).tobytes(), np.uint8)
        with pytest.raises(ValueError, match="stream overrun"):
            O.rans_decode(b)
        with pytest.raises(qa.QphError, match="stream overrun"):
            gpu_decode(b)


def test_large_chunked_q8_blob():
    """a 40 MiB q8-like blob coded as qpack-pack codes it (16 MiB chunks): 3 planes of up to 16M symbols each"""
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.02, 40 << 20)
    raw = np.clip(np.round(w / 0.0006), -127, 127).astype(np.int8).view(np.uint8)
    C = O.PACK_CHUNK
    blob = O.rans_assemble_chunked(len(raw), C, [O.rans_encode(raw[o:o + C], 1, 1) for o in range(0, len(raw), C)])
    out, ms = qa.kernel_rans_decode(blob)
    print(f"rans 40 MiB: {len(blob) / 2**20:.1f} MiB coded, decode {ms:.1f} ms ({len(raw) / ms / 1e6:.2f} GB/s)", flush=True)
    np.testing.assert_array_equal(out, raw)


@pytest.mark.parametrize("cfg", ["mini", "mini_q4m"])
def test_qpack3_model_equals_qpack2(cfg, synth, tmp_path):
    src = synth(cfg)
    dst = str(tmp_path / "m3.qpack")
    assert qa.pack(src, dst, 4) > 0
    toks = list(range(3, 40))
    a = qa.HipLlama.load(src, 128)
    b = qa.HipLlama.load(dst, 128)
    st = b.load_stats()
    assert st["planes"] > 0 and st["raw_bytes"] > st["coded_bytes"] > 0 and st["rounds"] >= 1
    assert a.load_stats()["planes"] == 0
    np.testing.assert_array_equal(a.prefill(toks, 1), b.prefill(toks, 1))
    np.testing.assert_array_equal(a.greedy_run(7, 24), b.greedy_run(7, 24))
    a.close(); b.close()


def test_create_with_coded_tensors(synth, tmp_path):
    """qph_create with the tensors of a QPACK3 file passed still coded (qph_tensor data_coded / scale_coded), the path a
    caller with its own container reader takes: the same logits and greedy stream as qph_load of the QPACK2 file"""
    import ctypes as C
    import json
    import struct
    from qpack_amd._lib import Config, Tensor, check, lib
    src = synth("mini_q4m")
    dst = str(tmp_path / "m3.qpack")
    qa.pack(src, dst, 2)
    raw = open(dst, "rb").read()
    n = struct.unpack("<I", raw[8:12])[0]
    toc = {}
    for i in range(n):
        e = raw[16 + 72 * i:16 + 72 * (i + 1)]
        toc[e[:56].rstrip(b"\0").decode()] = struct.unpack("<QQ", e[56:72])
    blob = lambda name: raw[toc[name][0]:toc[name][0] + toc[name][1]]   # noqa: E731
    man, cfgj = json.loads(blob("manifest.json")), json.loads(blob("config.json"))
    coded = set(man["encoded"])
    keep, ts = [], []
    for e in man["tensors"]:
        shape = e["shape"]
        rows, cols = (shape[0], shape[1]) if len(shape) == 2 else (shape[0], 1)
        kind = {"q8": qa.QPH_Q8, "q4": qa.QPH_Q4, "f32": qa.QPH_F32}[e["kind"]]
        d = C.create_string_buffer(blob(e["blob"]), toc[e["blob"]][1])
        s = C.create_string_buffer(blob(e["scale"]), toc[e["scale"]][1]) if "scale" in e else None
        keep += [d, s, e["name"].encode()]
        t = Tensor(name=keep[-1], kind=kind, rows=rows, cols=cols, data=C.cast(d, C.c_void_p),
                   scale=C.cast(s, C.c_void_p) if s else None,
                   data_coded=toc[e["blob"]][1] if e["blob"] in coded else 0,
                   scale_coded=toc[e["scale"]][1] if "scale" in e and e["scale"] in coded else 0)
        ts.append(t)
    assert any(t.data_coded for t in ts) and any(t.scale_coded for t in ts)
    cfg = Config(hidden=cfgj["hidden_size"], layers=cfgj["num_hidden_layers"], heads=cfgj["num_attention_heads"],
                 kv_heads=cfgj["num_key_value_heads"], head_dim=cfgj["head_dim"], ffn=cfgj["intermediate_size"],
                 vocab=cfgj["vocab_size"], tied=int(cfgj["tie_embeddings"]), qkv_bias=int(cfgj["qkv_bias"]), max_pos=cfgj["max_position_embeddings"],
                 rms_eps=cfgj["rms_norm_eps"], rope_theta=cfgj["rope_theta"])
    arr = (Tensor * len(ts))(*ts)
    h = C.c_void_p()
    check(lib().qph_create(C.byref(cfg), arr, len(ts), 128, C.byref(h)))
    m = qa.HipLlama(h.value)
    del keep, arr   # the library holds its own copies in HBM
    ref = qa.HipLlama.load(src, 128)
    toks = list(range(11, 50))
    np.testing.assert_array_equal(m.prefill(toks, 1), ref.prefill(toks, 1))
    np.testing.assert_array_equal(m.greedy_run(3, 20), ref.greedy_run(3, 20))
    assert m.load_stats()["planes"] > 0
    m.close(); ref.close()
