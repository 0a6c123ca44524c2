"""Device top-M of the logits (qph_step_topk / qph_prefill_topk / qph_kernel_topk) against the oracle's restatement of
the reference sampler's candidate selection (or_top_m: top_m + sort, /root/reference/src/sampler.cpp:12-27, :41-42,
pinned in tests/test_oracle.py against the compiled reference's Sampler and a stable numpy sort on (-value, index)):
the M largest values, value descending, the lower index first among equal values; exact equality of indices and
values is required."""
import numpy as np
import pytest

import oracle as O
import qpack_amd as qa

pytestmark = pytest.mark.gpu


def expect_topk(x, M):
    return O.top_m(x, M)


def check(x, M):
    idx, val = qa.kernel_topk(x, M)
    ei, ev = expect_topk(x, M)
    np.testing.assert_array_equal(idx, ei)
    np.testing.assert_array_equal(val, ev)


@pytest.mark.parametrize("n,M", [(n, M) for n in [1, 5, 4095, 4096, 4097, 8195, 151936] for M in [1, 7, 64, 512] if M <= n])
def test_topk_random(n, M):
    rng = np.random.default_rng(n * 1000 + M)
    print(f"topk n={n} M={M}", flush=True)
    check(rng.standard_normal(n).astype(np.float32) * 4, M)


@pytest.mark.parametrize("M", [1, 40, 512])
def test_topk_ties_and_specials(M):
    rng = np.random.default_rng(M)
    n = 20000
    x = np.round(rng.standard_normal(n) * 2) / 4           # few distinct values: long runs of equal values
    x = x.astype(np.float32)
    check(x, M)
    x[::7] = 0.0
    x[3::7] = -0.0                                          # equal to +0: the index decides
    x[100] = np.inf
    x[200] = -np.inf
    x[5000:5003] = np.float32(1e30)
    check(x, M)
    check(np.zeros(n, np.float32), M)                       # all equal: the first M indices
    check(-np.ones(n, np.float32), M)


def test_topk_rejects_bad_sizes():
    for n, M in ((100, 0), (100, 101), (600, 513)):
        with pytest.raises(qa.QphError):
            qa.kernel_topk(np.zeros(n, np.float32), M)


@pytest.mark.parametrize("cfg", ["mini", "mini_q4m"])
def test_step_and_prefill_topk_match_logits(cfg, synth):
    path = synth(cfg)
    gpu = qa.HipLlama.load(path, max_ctx=128)
    rng = np.random.default_rng(9)
    toks = rng.integers(0, gpu.vocab(), 40).astype(np.int32)
    lg = gpu.prefill(toks, 1)
    gpu.reset()
    idx, val = gpu.prefill_topk(toks, 64)
    ei, ev = expect_topk(lg, 64)
    np.testing.assert_array_equal(idx, ei)
    np.testing.assert_array_equal(val, ev)
    assert gpu.pos() == 40
    for t in rng.integers(0, gpu.vocab(), 5):
        p = gpu.pos()
        lg = gpu.step(int(t), 1)
        assert gpu.rewind(p)
        idx, val = gpu.step_topk(int(t), 40)
        ei, ev = expect_topk(lg, 40)
        np.testing.assert_array_equal(idx, ei)
        np.testing.assert_array_equal(val, ev)
        assert gpu.pos() == p + 1
    # greedy agreement: the top-1 of a step is the greedy pick
    p = gpu.pos()
    g = gpu.greedy_run(3, 1)
    assert gpu.rewind(p)
    idx, _ = gpu.step_topk(3, 1)
    assert idx[0] == g[0]
    gpu.close()
