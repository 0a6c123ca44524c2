"""Pins of the CPU oracle (oracle/oracle.c), CPU only.

Each oracle function is checked against something independent of its own formula:
  - golden vectors written by the reference compiled from its own sources (tests/golden/, make_golden.py);
  - the live reference library oracle/_ref/libqpref.so where it is built (this container);
  - brute force / closed forms in numpy (integer sums, quantisation, fp16 rounding, exp accuracy).
"""
import json
import os

import numpy as np
import pytest

import oracle as O
import qpack_amd as qa

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def gold(name):
    with open(os.path.join(GOLD, name + ".json")) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def kern():
    return np.load(os.path.join(GOLD, "kernels.npz"))


# ------------------------------------------------------------------ closed forms and brute force
def test_f16_rounding_matches_numpy():
    """or_f32_to_f16 is IEEE round-to-nearest-even: numpy's float16 cast is an independent implementation"""
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.normal(0, 1, 20000), rng.normal(0, 1e4, 5000), rng.normal(0, 1e-5, 5000),
                        [0.0, -0.0, 65504, 65519.99, 65520, 1e9, -1e9, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 6e-8, np.inf, -np.inf]])
    x = x.astype(np.float32)
    got = O.f32_to_f16(x)
    np.testing.assert_array_equal(got, x.astype(np.float16).view(np.uint16))
    h = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    h = h[(h & 0x7c00) != 0x7c00]   # finite halves: exact round trip
    back = np.array([O.olib().or_f16_to_f32(int(v)) for v in h[::7]], np.float32)
    np.testing.assert_array_equal(back, h[::7].view(np.float16).astype(np.float32))


def numpy_quant(x):
    """quant_rows (/root/reference/src/kernels.cpp:17-31) written out in numpy float32"""
    x = x.astype(np.float32)
    nb = (len(x) + 127) // 128
    q = np.empty(len(x), np.int16)
    bs = np.empty(nb, np.float32)
    for b in range(nb):
        v = x[128 * b:128 * b + 128]
        mx = np.float32(np.abs(v).max())
        isx = np.float32(32767) / mx if mx > 0 else np.float32(0)
        bs[b] = mx / np.float32(32767)
        q[128 * b:128 * b + 128] = np.rint((v * isx).astype(np.float32)).astype(np.int16)
    return q, bs


def test_quant_act_brute_force():
    rng = np.random.default_rng(1)
    for cols in (128, 896, 4096, 1000):
        x = rng.normal(0, 1, cols).astype(np.float32)
        x[:128] = 0 if cols > 128 else x[:128]
        x[min(200, cols - 1)] = 1e3
        xq, bs = O.quant_act(x)
        q2, b2 = numpy_quant(x)
        np.testing.assert_array_equal(xq, q2)
        np.testing.assert_array_equal(bs, b2)
        assert np.abs(xq).max() == 32767


def test_block_and_group_sums_brute_force():
    rng = np.random.default_rng(2)
    q = rng.integers(-127, 128, (17, 896)).astype(np.int8)
    xq = rng.integers(-32767, 32768, 896).astype(np.int16)
    ref = (q.astype(np.int64) * xq.astype(np.int64)).reshape(17, 7, 128).sum(2)
    np.testing.assert_array_equal(O.block_sums_q8(q, xq), ref)
    q4 = rng.integers(0, 256, (9, 448)).astype(np.uint8)
    g = q4.reshape(9, 28, 16)
    w = np.concatenate([(g & 15).astype(np.int64) - 8, (g >> 4).astype(np.int64) - 8], axis=2)   # [rows, groups, 32]
    ref4 = (w * xq.astype(np.int64).reshape(28, 32)[None]).sum(2)
    np.testing.assert_array_equal(O.group_sums_q4(q4, xq), ref4)


def test_exp_accuracy():
    """exp256 (kernels_x86.cpp:406-417) against float64 exp: ~1e-6 relative for |x| <= 20 (softmax / SiLU inputs), the
    Cody-Waite reduction grows to ~4e-6 near the clamp; the exact bits are pinned by the golden vectors"""
    x = np.linspace(-80, 80, 10001).astype(np.float32)
    y = O.exp_v(x)
    rel = np.abs(y.astype(np.float64) - np.exp(x.astype(np.float64))) / np.exp(x.astype(np.float64))
    assert rel.max() < 5e-6
    assert rel[np.abs(x) <= 20].max() < 1.2e-6


def test_rows_q8_equals_scaled_block_sums():
    """rows_q8 is sum_b bs[b] * isum_b times the row scale: compare with float64 evaluation"""
    rng = np.random.default_rng(3)
    q = rng.integers(-127, 128, (64, 1024)).astype(np.int8)
    s = (rng.random(64) * 0.01).astype(np.float32)
    x = rng.normal(0, 1, 1024).astype(np.float32)
    xq, bs = O.quant_act(x)
    y = O.rows_q8(q, s, xq, bs)
    exact = (O.block_sums_q8(q, xq).astype(np.float64) * bs.astype(np.float64)).sum(1) * s
    assert np.allclose(y, exact, rtol=1e-5, atol=1e-7)


# ------------------------------------------------------------------ golden vectors of the compiled reference
@pytest.mark.parametrize("shape", ["48x1024", "33x896"])
def test_matvec_matmul_golden(kern, shape):
    k = "q8_" + shape
    np.testing.assert_array_equal(O.matvec(O.OR_Q8, kern[k + "_q"], kern[k + "_s"], kern[k + "_x"]), kern[k + "_y"])
    np.testing.assert_array_equal(O.matmul(O.OR_Q8, kern[k + "_q"], kern[k + "_s"], kern[k + "_X"]), kern[k + "_Y"])
    k = "q4_" + shape
    np.testing.assert_array_equal(O.matvec(O.OR_Q4, kern[k + "_q"], kern[k + "_s"], kern[k + "_x"]), kern[k + "_y"])
    np.testing.assert_array_equal(O.matmul(O.OR_Q4, kern[k + "_q"], kern[k + "_s"], kern[k + "_X"]), kern[k + "_Y"])


@pytest.mark.parametrize("shape", ["48x1024", "33x896", "9x1000"])
def test_q1_matvec_matmul_golden(kern, shape):
    k, cols = "q1_" + shape, int(shape.split("x")[1])
    np.testing.assert_array_equal(O.matvec(O.OR_Q1, kern[k + "_q"], kern[k + "_s"], kern[k + "_x"], cols), kern[k + "_y"])
    np.testing.assert_array_equal(O.matmul(O.OR_Q1, kern[k + "_q"], kern[k + "_s"], kern[k + "_X"], cols), kern[k + "_Y"])


def test_q1_group_sums_brute_force():
    """exact int32 per (row, 128-column group) against numpy on the unpacked sign bits, partial last group included"""
    rng = np.random.default_rng(8)
    for rows, cols in [(3, 128), (5, 1000), (4, 4096)]:
        G = (cols + 127) // 128
        q = rng.integers(0, 256, (rows, G * 16)).astype(np.uint8)
        xq = rng.integers(-32767, 32768, cols).astype(np.int16)
        sign = (np.unpackbits(q, axis=1, bitorder="little").astype(np.int64) * 2 - 1)[:, :cols]
        xp = np.zeros(G * 128, np.int64); xp[:cols] = xq
        brute = (np.pad(sign, ((0, 0), (0, G * 128 - cols))).reshape(rows, G, 128) * xp.reshape(1, G, 128)).sum(2)
        np.testing.assert_array_equal(O.group_sums_q1(q, xq, cols), brute)


def test_elementwise_golden(kern):
    np.testing.assert_array_equal(O.rmsnorm(kern["rms_x"], kern["rms_w"], 1e-6), kern["rms_out"])
    np.testing.assert_array_equal(O.silu_mul(kern["silu_g"], kern["silu_u"]), kern["silu_out"])
    np.testing.assert_array_equal(O.exp_v(kern["exp_x"]), kern["exp_out"])


@pytest.mark.parametrize("name", ["mini", "mini128", "mini_q4", "mini_q4m", "c1", "mini_q1", "mini_q1m", "mini_q4mb",
                                  "mini_q4h"])
def test_model_golden(name, tmp_path):
    """prefill logits sample and the whole greedy stream are bit-identical to the reference's"""
    fx = gold(name)
    path = str(tmp_path / f"{name}.qpack")
    qa.write_synthetic(name, path, seed=fx["seed"])
    o = O.Oracle(path, fx["max_ctx"])
    lg = o.prefill(np.array(fx["prompt"], np.int32), 1)
    np.testing.assert_array_equal(lg[fx["prefill_sample_idx"]], np.float32(fx["prefill_sample"]))
    assert int(np.argmax(lg)) == fx["first_token"]
    g = o.greedy_run(fx["first_token"], len(fx["greedy"]))
    np.testing.assert_array_equal(g, fx["greedy"])
    assert o.pos() == fx["pos_after"]
    o.close()


# ------------------------------------------------------------------ live reference (where it is built)
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref/libqpref.so not built (needs /root/reference)")


@needs_ref
@pytest.mark.parametrize("name", ["mini_q4m", "mini128", "mini_q1m"])
def test_model_matches_live_reference(name, tmp_path):
    path = str(tmp_path / f"{name}.qpack")
    qa.write_synthetic(name, path, seed=77)
    ref, o = O.Ref(path, 300), O.Oracle(path, 300)
    toks = np.random.default_rng(5).integers(0, ref.vocab(), 67).astype(np.int32)
    np.testing.assert_array_equal(ref.prefill(toks, 1), o.prefill(toks, 1))
    for t in (3, 9, 27):
        np.testing.assert_array_equal(ref.step(t, 1), o.step(t, 1))
    np.testing.assert_array_equal(ref.step(4, 2), o.step(4, 2))
    k, v = o.kv_cache()
    snap = np.frombuffer(ref.snapshot(), np.uint8)
    L, kvd, n = o.cfg.L, o.cfg.nkv * o.cfg.hd, ref.pos()
    assert snap[:4].view(np.int32)[0] == n
    body = snap[4:].view(np.uint16).reshape(L, 2, n, kvd)
    np.testing.assert_array_equal(body[:, 0], k[:, :n])
    np.testing.assert_array_equal(body[:, 1], v[:, :n])


def _topk_cases():
    rng = np.random.default_rng(77)
    cases = []
    for V, M in ((151936, 40), (128256, 512), (1000, 250), (1000, 251), (5000, 1), (8200, 64), (17, 3)):
        cases.append((rng.standard_normal(V).astype(np.float32) * 3, M))
    x = (np.round(rng.standard_normal(60000) * 2) / 4).astype(np.float32)   # long runs of equal values
    x[::7] = 0.0; x[3::7] = -0.0; x[100] = np.inf; x[200] = -np.inf
    cases += [(x, 1), (x, 40), (x, 512), (np.zeros(9000, np.float32), 33)]
    return cases


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref/libqpref.so not built")
def test_top_m_matches_reference_sampler():
    """or_top_m against the compiled reference's own sampler (Sampler::dist with top_k = M) and against the textbook
    order (a stable sort on (-value, index)), including ties, -0 / +0, infinities and M >= V / 4"""
    for x, M in _topk_cases():
        idx, val = O.top_m(x, M)
        np.testing.assert_array_equal(idx, O.ref_sampler_topk(x, M))
        np.testing.assert_array_equal(idx, np.lexsort((np.arange(len(x)), -x.astype(np.float64)))[:M])
        np.testing.assert_array_equal(val, x[idx])


@pytest.mark.parametrize("name", ["mini", "mini_q4m", "c1", "c2", "c3"])
def test_fixture_prefill_all_equals_steps(name):
    """the reference's own contract, read off its fixtures: prefill_all under ExactBatches (qpack.h:106-108, :152)
    gives every position's logits bit-identical to stepping the same tokens (per-position hashes equal the decode
    steps' hashes)"""
    with open(os.path.join(GOLD, name + ".json")) as f:
        fx = json.load(f)
    pa = fx["prefill_all"]
    assert pa["tokens"] == [fx["first_token"]] + fx["greedy"][:7]
    assert pa["hash"] == fx["step_hash"][:8]
    assert pa["argmax"] == fx["greedy"][:8]
