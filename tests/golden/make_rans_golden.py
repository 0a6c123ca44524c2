"""Writes tests/golden/rans.npz: QPACK3 rANS blobs made by the reference codec compiled from its own sources
(qp::rans::encode / decode of /root/reference/include/qpack/rans.h, through oracle/_ref/libqpref.so).  Run in the build
container:

    python tests/golden/make_rans_golden.py

Cases: seeded raw byte strings of several lengths (0 .. 20000) and statistics (uniform, narrow Gaussian, constant,
two-valued, quantised N(0, 0.02) weights, q4 nibbles), each coded as codec 1 with 1 / 2 / 3 / 4 planes or as codec 2,
stored as (raw, blob).  Error cases: malformed blobs derived from a good one with the message the reference decoder
throws for each (truncated plane, bad frequency table, unknown codec, stream overrun, short blob).
"""
import ctypes as C
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle as O  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def raw_case(rng, kind, n):
    if kind == "uniform":
        return rng.integers(0, 256, n, dtype=np.uint8)
    if kind == "narrow":
        return np.clip(rng.normal(128, 3, n), 0, 255).astype(np.uint8)
    if kind == "const":
        return np.full(n, 0x5a, np.uint8)
    if kind == "two":
        return np.where(rng.random(n) < 0.999, 7, 200).astype(np.uint8)
    if kind == "q8":   # quantise_q8 of N(0, 0.02) rows (qpack-quantize's rule: round(w / (max|w| / 127)))
        w = rng.normal(0, 0.02, (max(n // 64, 1), 64))
        q = np.round(w / (np.abs(w).max(1, keepdims=True) / 127)).astype(np.int8)
        return q.reshape(-1)[:n].view(np.uint8).copy()
    if kind == "q4":   # two nibbles of q + 8, q in [-8, 7] concentrated near 0
        q = np.clip(np.round(rng.normal(0, 2.2, 2 * n)), -8, 7).astype(np.int64) + 8
        return (q[0::2] | (q[1::2] << 4)).astype(np.uint8)
    raise ValueError(kind)


def main():
    L = O.rlib(1)

    def enc(raw, codec, planes):
        cap = 4 * len(raw) + 4096
        out = np.empty(cap, np.uint8)
        n = C.c_int64()
        if L.qpref_rans_encode(O._p(raw), len(raw), codec, planes, O._p(out), cap, C.byref(n)):
            raise RuntimeError(L.qpref_error().decode())
        return out[:n.value].copy()

    def dec_err(blob):
        n = max(L.qpref_rans_raw_size(O._p(blob), len(blob)), 0)
        out = np.zeros(n + 16, np.uint8)
        return "" if L.qpref_rans_decode(O._p(blob), len(blob), O._p(out)) == 0 else L.qpref_error().decode()

    rng = np.random.default_rng(20261201)
    arrays, meta = {}, []
    plans = [(1, 1), (1, 2), (1, 3), (1, 4), (2, 1)]
    i = 0
    for kind, sizes in [("uniform", [0, 1, 2, 3, 5, 8, 64, 1000, 3001]), ("narrow", [4, 17, 4096, 9000]),
                        ("const", [1, 9, 3000]), ("two", [6000]), ("q8", [8192]), ("q4", [6144])]:
        for n in sizes:
            raw = raw_case(rng, kind, n)
            for codec, planes in plans:
                if kind == "q4" and codec == 1 and planes > 1:
                    continue
                blob = enc(raw, codec, planes)
                arrays[f"raw{i}"], arrays[f"blob{i}"] = raw, blob
                meta.append((i, codec, planes, n))
                i += 1
    # malformed blobs (from a narrow codec 1 blob of 4096 bytes) and the reference's message for each
    good = enc(raw_case(rng, "narrow", 4096), 1, 1)
    bad = {}
    t = good.copy(); t[6:10] = np.frombuffer(np.uint32(len(good)).tobytes(), np.uint8); bad["comp_len_past_end"] = t
    t = good.copy(); t[10] ^= 1; bad["freq_sum"] = t
    t = good.copy(); t[0] = 9; bad["codec"] = t
    cl = int(np.frombuffer(good[6:10].tobytes(), np.uint32)[0])
    t = good.copy(); t[6:10] = np.frombuffer(np.uint32(cl - 64).tobytes(), np.uint8); bad["overrun"] = t
    bad["short"] = good[:4].copy()
    errs = []
    for k, b in bad.items():
        arrays[f"bad_{k}"] = b
        errs.append((k, dec_err(b)))
    arrays["meta"] = np.array(meta, np.int64)
    arrays["errors"] = np.array([f"{k}\t{m}" for k, m in errs])
    np.savez_compressed(os.path.join(HERE, "rans.npz"), **arrays)
    print(f"{len(meta)} cases, errors: {errs}")


if __name__ == "__main__":
    main()
