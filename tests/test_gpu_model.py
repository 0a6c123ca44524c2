"""GPU parity of the whole token loop (qp::Model surface over the C ABI) against the oracle on small seeded models.

Bar: logits within max-abs 1e-2 and relative 1e-3 of the reference, identical greedy streams.
"""
import numpy as np
import pytest

import oracle as O
import qpack_amd as qa

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-2, 1e-3


def close(a, b):
    err = np.abs(a - b)
    return float(err.max()), bool(np.all(err <= np.maximum(ATOL, RTOL * np.abs(b))))


@pytest.mark.parametrize("cfg", ["mini", "mini128", "mini_q4", "mini_q4m"])
def test_decode_and_greedy_match_oracle(cfg, synth):
    path = synth(cfg)
    gpu = qa.HipLlama.load(path, max_ctx=256)
    orc = O.Oracle(path, max_ctx=256)
    rng = np.random.default_rng(3)
    toks = rng.integers(0, gpu.vocab(), 70).astype(np.int32)
    print(f"{cfg}: prefill 70", flush=True)
    lg, lo = gpu.prefill(toks, 1), orc.prefill(toks, 1)
    err, ok = close(lg, lo)
    assert ok, f"prefill logits max|d| {err}"
    for t in rng.integers(0, gpu.vocab(), 6):
        err, ok = close(gpu.step(int(t), 1), orc.step(int(t), 1))
        assert ok, f"step logits max|d| {err}"
    g, o = gpu.greedy_run(int(np.argmax(lg)), 48), orc.greedy_run(int(np.argmax(lo)), 48)
    np.testing.assert_array_equal(g, o)
    assert gpu.pos() == orc.pos() == 70 + 6 + 48
    gpu.close(); orc.close()


def test_want_hidden_and_state_only(synth):
    path = synth("mini")
    gpu = qa.HipLlama.load(path, max_ctx=64)
    orc = O.Oracle(path, max_ctx=64)
    for t in (1, 2, 3):
        assert gpu.step(t, 0) is None
        orc.step(t, 0)
    err, ok = close(gpu.step(4, 2), orc.step(4, 2))
    assert ok, err
    assert gpu.pos() == 4


def test_snapshot_restore_rewind(synth):
    path = synth("mini128")
    gpu = qa.HipLlama.load(path, max_ctx=128)
    toks = np.arange(1, 20, dtype=np.int32)
    gpu.prefill(toks, 0)
    snap = gpu.snapshot()
    assert len(snap) == 4 + 2 * 2 * 19 * 128 * 2
    a = gpu.step(7, 1)
    gpu2 = qa.HipLlama.load(path, max_ctx=128)
    gpu2.restore(snap)
    assert gpu2.pos() == 19
    np.testing.assert_array_equal(gpu2.step(7, 1), a)
    assert gpu.rewind(19) and not gpu.rewind(50)
    np.testing.assert_array_equal(gpu.step(7, 1), a)
    c = gpu.checkpoint()
    gpu.step(8, 0)
    gpu.rollback(c)
    assert gpu.pos() == 20


def test_errors_are_reported(synth):
    path = synth("mini")
    gpu = qa.HipLlama.load(path, max_ctx=8)
    with pytest.raises(qa.QphError, match="out of range"):
        gpu.step(10**6, 1)
    gpu.prefill(np.arange(8, dtype=np.int32), 0)
    with pytest.raises(qa.QphError, match="context window full"):
        gpu.step(1, 1)
    assert len(gpu.greedy_run(1, 4)) == 0
    with pytest.raises(qa.QphError):
        qa.HipLlama.load("/nonexistent.qpack")
