"""Writes the golden fixtures of tests/golden/ from the reference engine compiled from its own sources
(oracle/_ref/libqpref.so, built by oracle/Makefile from /root/reference).  Run in the build container:

    python tests/golden/make_golden.py

Model fixtures (<cfg>.json): a seeded synthetic QPACK2 file (qpack_amd.write_synthetic, regenerated bit-identically from
the seed by the tests), a seeded prompt, and what the reference computes on it with the qpack-bench protocol
(/root/reference/tools/qpack-bench.cpp:40-45): prefill(prompt) -> logits, then greedy decoding by step(tok, 1) + argmax
(the default Model::greedy_run, /root/reference/include/qpack/qpack.h:143-149).  Stored: the greedy stream, the top-2 gap
of every step, top-5 ids / logits of the prefill and of the first decode steps, and a fixed sample of the prefill logits
with their float64 sum.

Kernel fixtures (kernels.npz): seeded q8 / q4 matrices and activations with edge cases (zero block, outliers), the
reference's matvec output for each (qp::matvec: quant_rows + rows_q8 / rows_q4), its tiled matmul output (mm_q8 /
mm_q4, 6 vectors), rmsnorm and silu_mul outputs.
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle as O  # noqa: E402
import qpack_amd as qa  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
TMP = os.environ.get("TMPDIR", "/tmp")

# name: (prompt tokens, greedy tokens, max_ctx)
MODELS = {
    "mini": (70, 64, 256),
    "mini128": (131, 64, 256),
    "mini_q4": (70, 64, 256),
    "mini_q4m": (100, 64, 256),
    "c1": (32, 128, 168),
    "c2": (512, 256, 776),
    "mini_q1": (70, 64, 256),
    "mini_q1m": (70, 64, 256),
    "mini_q4mb": (70, 64, 256),
    "mini_q4h": (70, 64, 256),
}
SEED = 1234
PROMPT_SEED = 99


def prompt_for(name, vocab):
    return np.random.default_rng(PROMPT_SEED).integers(0, vocab, MODELS[name][0]).astype(np.int32)


def top(l, k):
    i = np.argsort(-l, kind="stable")[:k]
    return i.tolist(), l[i].astype(float).tolist()


def model_fixture(name):
    n_prompt, n_gen, ctx = MODELS[name]
    path = os.path.join(TMP, f"golden_{name}.qpack")
    qa.write_synthetic(name, path, seed=SEED)
    ref = O.Ref(path, ctx)
    V = ref.vocab()
    toks = prompt_for(name, V)
    lg = ref.prefill(toks, 1)
    pi, pv = top(lg, 10)
    sample_idx = np.arange(0, V, max(1, V // 512))
    tok = int(np.argmax(lg))
    stream, gaps, tops = [], [], []
    for i in range(n_gen):
        l = ref.step(tok, 1)
        s = np.sort(l)
        gaps.append(float(s[-1] - s[-2]))
        if i < 16:
            tops.append(top(l, 5))
        tok = int(np.argmax(l))
        stream.append(tok)
    fx = dict(config=name, seed=SEED, prompt_seed=PROMPT_SEED, max_ctx=ctx, prompt=toks.tolist(), prefill_top10=[pi, pv],
              prefill_sample_idx=sample_idx.tolist(), prefill_sample=lg[sample_idx].astype(float).tolist(),
              prefill_sum=float(lg.astype(np.float64).sum()), first_token=int(np.argmax(lg)), greedy=stream,
              greedy_top2_gap=gaps, decode_top5=tops, pos_after=int(ref.pos()))
    ref.close()
    os.remove(path)
    with open(os.path.join(HERE, f"{name}.json"), "w") as f:
        json.dump(fx, f)
    print(f"{name}: stream {stream[:12]}..., min top-2 gap {min(gaps):.3g}", flush=True)


def act_vector(rng, cols):
    x = rng.normal(0, 1, cols).astype(np.float32)
    x[128:256] = 0
    x[5] = 300.0
    x[-60] = -7.25
    return x


def kernel_fixture():
    rng = np.random.default_rng(2024)
    L = O.rlib()
    out = {}
    for rows, cols in [(48, 1024), (33, 896)]:
        q = rng.integers(-127, 128, (rows, cols)).astype(np.int8)
        s = (rng.random(rows) * 0.01 + 1e-4).astype(np.float32)
        x = act_vector(rng, cols)
        y = np.empty(rows, np.float32)
        assert L.qpref_matvec(0, q.ctypes.data, s.ctypes.data, rows, cols, O._f(x), O._f(y)) == 0
        X = np.stack([act_vector(rng, cols) * (i + 1) for i in range(6)]).astype(np.float32)
        Y = np.empty((6, rows), np.float32)
        assert L.qpref_matmul(0, q.ctypes.data, s.ctypes.data, rows, cols, O._f(X), 6, O._f(Y), 0) == 0
        k = f"q8_{rows}x{cols}"
        out.update({k + "_q": q, k + "_s": s, k + "_x": x, k + "_y": y, k + "_X": X, k + "_Y": Y})
        q4 = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
        s4 = (rng.random((rows, cols // 32)) * 0.01 + 1e-4).astype(np.float16).view(np.uint16)
        y4 = np.empty(rows, np.float32)
        assert L.qpref_matvec(1, q4.ctypes.data, s4.ctypes.data, rows, cols, O._f(x), O._f(y4)) == 0
        Y4 = np.empty((6, rows), np.float32)
        assert L.qpref_matmul(1, q4.ctypes.data, s4.ctypes.data, rows, cols, O._f(X), 6, O._f(Y4), 0) == 0
        k = f"q4_{rows}x{cols}"
        out.update({k + "_q": q4, k + "_s": s4, k + "_x": x, k + "_y": y4, k + "_X": X, k + "_Y": Y4})
    x = rng.normal(0, 3, 1000).astype(np.float32)
    w = rng.normal(1, 0.1, 1000).astype(np.float32)
    o = np.empty_like(x)
    L.qpref_rmsnorm(O._f(x), O._f(w), 1000, np.float32(1e-6), O._f(o))
    g = rng.normal(0, 4, 1003).astype(np.float32)
    u = rng.normal(0, 1, 1003).astype(np.float32)
    gs = g.copy()
    L.qpref_silu_mul(O._f(gs), O._f(u), 1003)
    e = rng.uniform(-100, 100, 1005).astype(np.float32)
    ev = np.empty_like(e)
    L.qpref_exp_v(O._f(e), O._f(ev), 1005)
    out.update(dict(rms_x=x, rms_w=w, rms_out=o, silu_g=g, silu_u=u, silu_out=gs, exp_x=e, exp_out=ev))
    # q1 (rows_q1 / mm_q1): sign bits and fp16 group scales; 1000 columns end in a partial group
    r1 = np.random.default_rng(2025)
    for rows, cols in [(48, 1024), (33, 896), (9, 1000)]:
        G = (cols + 127) // 128
        q1 = r1.integers(0, 256, (rows, G * 16)).astype(np.uint8)
        s1 = (r1.random((rows, G)) * 0.01 + 1e-4).astype(np.float16).view(np.uint16)
        x1 = act_vector(r1, cols)
        y1 = np.empty(rows, np.float32)
        assert L.qpref_matvec(3, q1.ctypes.data, s1.ctypes.data, rows, cols, O._f(x1), O._f(y1)) == 0
        X1 = np.stack([act_vector(r1, cols) * (i + 1) for i in range(6)]).astype(np.float32)
        Y1 = np.empty((6, rows), np.float32)
        assert L.qpref_matmul(3, q1.ctypes.data, s1.ctypes.data, rows, cols, O._f(X1), 6, O._f(Y1), 0) == 0
        k = f"q1_{rows}x{cols}"
        out.update({k + "_q": q1, k + "_s": s1, k + "_x": x1, k + "_y": y1, k + "_X": X1, k + "_Y": Y1})
    np.savez_compressed(os.path.join(HERE, "kernels.npz"), **out)
    print("kernels.npz written", flush=True)


if __name__ == "__main__":
    O.rlib(int(os.environ.get("QPREF_THREADS", "8")))
    kernel_fixture()
    for name in (sys.argv[1:] or MODELS):
        model_fixture(name)
