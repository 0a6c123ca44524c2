"""GPU parity of the matvec kernel (the decode hot path) against the oracle, through the C ABI.

Bar: int16 activations, block scales and int32 accumulators bit-exact; q8 outputs bit-identical to rows_q8
(/root/reference/src/kernels_x86.cpp:55-71); q4 outputs within 2e-6 relative to the sum of |group terms| (the q4
float order is a per-lane chain + wave tree instead of rows_q4's 8-lane split).
"""
import numpy as np
import pytest

import oracle as O
import qpack_amd as qa

pytestmark = pytest.mark.gpu


def act_vector(rng, cols):
    """N(0,1) activations with the cases quant_rows must get right: an all-zero block, outliers, a single spike"""
    x = rng.normal(0, 1, cols).astype(np.float32)
    x[128:256] = 0                      # all-zero block -> scale 0
    x[5] = 300.0                        # outlier coarsens only its own block
    x[-128:] = 0; x[-60] = -7.25        # one non-zero value in a block
    x[300:310] = 1e-30                  # tiny values
    return x


def q8_matrix(rng, rows, cols):
    q = rng.integers(-127, 128, (rows, cols)).astype(np.int8)
    q[0, :] = 127; q[min(1, rows - 1), :] = -127       # extreme rows
    s = (rng.random(rows).astype(np.float32) * 0.01 + 1e-4).astype(np.float32)
    return q, s


@pytest.mark.parametrize("rows,cols", [(1000, 4096), (513, 896), (300, 14336), (64, 18944), (7, 128), (4864, 896)])
def test_matvec_q8_bit_exact(rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    q, s = q8_matrix(rng, rows, cols)
    x = act_vector(rng, cols)
    print(f"q8 matvec rows={rows} cols={cols}", flush=True)
    y, sums, xq, bs = qa.kernel_matvec(qa.QPH_Q8, q, s, x)
    xq_o, bs_o = O.quant_act(x)
    np.testing.assert_array_equal(xq, xq_o)
    np.testing.assert_array_equal(bs, bs_o)
    np.testing.assert_array_equal(sums, O.block_sums_q8(q, xq_o))
    np.testing.assert_array_equal(y, O.rows_q8(q, s, xq_o, bs_o))


@pytest.mark.parametrize("rows,cols", [(1000, 4096), (257, 896), (300, 18944), (9, 128), (3584, 3584)])
def test_matvec_q4_exact_sums(rows, cols):
    rng = np.random.default_rng(rows * 11 + cols)
    q = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
    s = (rng.random((rows, cols // 32)) * 0.01 + 1e-4).astype(np.float16).view(np.uint16)
    x = act_vector(rng, cols)
    print(f"q4 matvec rows={rows} cols={cols}", flush=True)
    y, sums, xq, bs = qa.kernel_matvec(qa.QPH_Q4, q, s, x)
    xq_o, bs_o = O.quant_act(x)
    np.testing.assert_array_equal(xq, xq_o)
    gs = O.group_sums_q4(q, xq_o)
    np.testing.assert_array_equal(sums, gs)
    y_o = O.rows_q4(q, s, xq_o, bs_o)
    comb = s.view(np.float16).astype(np.float32) * np.repeat(bs_o, 4)[None, :]
    mag = np.abs(comb * gs).sum(1)
    assert np.all(np.abs(y - y_o) <= 2e-6 * mag + 1e-30), float(np.max(np.abs(y - y_o) / (mag + 1e-30)))


@pytest.mark.parametrize("rows,cols", [(1000, 4096), (257, 896), (300, 18944), (9, 128), (4096, 14336), (14336, 4096)])
def test_matvec_q1_exact_sums(rows, cols):
    """q1 (rows_q1, kernels_x86.cpp:167-203): the exact int32 dot product of every (row, 128-column group) equals a
    brute-force numpy sum over the unpacked signs; y within 2e-6 of the summed magnitudes of the oracle's (fp32 order:
    per-lane fma over the groups, then the wave sum, instead of the reference's 8 AVX lanes)"""
    rng = np.random.default_rng(rows * 13 + cols)
    G = cols // 128
    q = rng.integers(0, 256, (rows, G * 16)).astype(np.uint8)
    s = (rng.random((rows, G)) * 0.01 + 1e-4).astype(np.float16).view(np.uint16)
    x = act_vector(rng, cols)
    print(f"q1 matvec rows={rows} cols={cols}", flush=True)
    y, sums, xq, bs = qa.kernel_matvec(qa.QPH_Q1, q, s, x)
    xq_o, bs_o = O.quant_act(x)
    np.testing.assert_array_equal(xq, xq_o)
    sign = np.unpackbits(q, axis=1, bitorder="little").astype(np.int64) * 2 - 1      # [rows, cols]: +1 / -1
    brute = (sign.reshape(rows, G, 128) * xq_o.astype(np.int64).reshape(1, G, 128)).sum(2)
    np.testing.assert_array_equal(sums, brute)
    np.testing.assert_array_equal(O.group_sums_q1(q, xq_o, cols), brute)
    y_o = O.rows_q1(q, s, xq_o, bs_o, cols)
    comb = s.view(np.float16).astype(np.float32) * bs_o[None, :]
    mag = np.abs(comb * brute).sum(1)
    assert np.all(np.abs(y - y_o) <= 2e-6 * mag + 1e-30), float(np.max(np.abs(y - y_o) / (mag + 1e-30)))


@pytest.mark.parametrize("rows,cols,B", [(1000, 4096, 200), (256, 896, 129), (300, 14336, 17), (7, 128, 1), (4864, 896, 64),
                                         (130, 512, 1024), (300, 896, 2048),
                                         (130, 512, 300)])
@pytest.mark.parametrize("kernel", ["16x16", "32x32"])
def test_matmul_q8_rows_equal_decode_arithmetic(rows, cols, B, kernel, monkeypatch):
    """batched prefill product (int8 MFMA, two activation planes), each of the two q8 kernels forced (QPH_GEMM): every
    token's row bit-identical to rows_q8 on that token's quantised activation - the decode step's arithmetic; ragged
    row / token counts exercise the tile edges"""
    monkeypatch.setenv("QPH_GEMM", "1" if kernel == "32x32" else "2")
    rng = np.random.default_rng(rows * 13 + cols + B)
    q, s = q8_matrix(rng, rows, cols)
    X = np.stack([act_vector(rng, cols) * rng.uniform(0.1, 10) for _ in range(B)]).astype(np.float32)
    X[B // 2] = 0                                   # an all-zero token
    print(f"q8 matmul {kernel} rows={rows} cols={cols} B={B}", flush=True)
    Y = qa.kernel_matmul(q, s, X)
    for b in range(B):
        xq, bs = O.quant_act(X[b])
        np.testing.assert_array_equal(Y[b], O.rows_q8(q, s, xq, bs), err_msg=f"token {b}")


@pytest.mark.parametrize("rows,cols,B", [(1000, 4096, 200), (257, 896, 129), (300, 18944, 17), (9, 128, 1), (3584, 3584, 64),
                                         (130, 512, 1024)])
def test_matmul_q4(rows, cols, B):
    """batched prefill product on q4 rows (int8 MFMA over unpacked nibbles, exact int32 group sums): every token's row
    against rows_q4 on that token's quantised activation, within 2e-6 of the summed term magnitudes (its own fp32
    order); ragged row / token counts exercise the tile edges"""
    rng = np.random.default_rng(rows * 17 + cols + B)
    q = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
    q[0] = 0x00; q[min(1, rows - 1)] = 0xff                    # extreme nibbles (-8, 7)
    s = (rng.random((rows, cols // 32)) * 0.01 + 1e-4).astype(np.float16).view(np.uint16)
    X = np.stack([act_vector(rng, cols) * rng.uniform(0.1, 10) for _ in range(B)]).astype(np.float32)
    X[B // 2] = 0
    print(f"q4 matmul rows={rows} cols={cols} B={B}", flush=True)
    Y = qa.kernel_matmul(q, s, X)
    for b in range(0, B, max(1, B // 40)):
        xq, bs = O.quant_act(X[b])
        gs = O.group_sums_q4(q, xq)
        comb = s.view(np.float16).astype(np.float32) * np.repeat(bs, 4)[None, :]
        mag = np.abs(comb * gs).sum(1)
        y_o = O.rows_q4(q, s, xq, bs)
        assert np.all(np.abs(Y[b] - y_o) <= 2e-6 * mag + 1e-30), (b, float(np.max(np.abs(Y[b] - y_o) / (mag + 1e-30))))


@pytest.mark.parametrize("kind", ["q8", "q4"])
@pytest.mark.parametrize("rows,cols,B", [(48, 1024, 6), (257, 896, 64), (300, 4096, 1), (130, 512, 27), (64, 14336, 5),
                                         (1000, 4096, 40)])
def test_matmul_reference_order_bit_exact(kind, rows, cols, B):
    """the reference-order products (qph_kernel_matmul_ref, the prompt products of set_order(1)): bit-identical to the
    oracle's matmul - mm_q8 / mm_q4 lane order for the first B - B % 4 vectors, rows_q8 / rows_q4 for the rest - which
    is pinned bit-exact to the reference's matmul (tests/test_oracle.py, tests/golden/kernels.npz)"""
    rng = np.random.default_rng(rows * 19 + cols + B)
    if kind == "q8":
        q, s = q8_matrix(rng, rows, cols)
        k = O.OR_Q8
    else:
        q = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
        s = (rng.random((rows, cols // 32)) * 0.01 + 1e-4).astype(np.float16).view(np.uint16)
        k = O.OR_Q4
    X = np.stack([act_vector(rng, cols) * rng.uniform(0.1, 10) for _ in range(B)]).astype(np.float32)
    print(f"reference-order {kind} matmul rows={rows} cols={cols} B={B}", flush=True)
    Y = qa.kernel_matmul(q, s, X, order=1)
    np.testing.assert_array_equal(Y, O.matmul(k, q, s, X))


def test_matmul_reference_order_golden():
    """the same products on the reference's own outputs (tests/golden/kernels.npz: its matmul of 6 vectors, and its
    matvec of one): q8, q4, and q1 (the reference order's q1 products, rows_q1 / mm_q1)"""
    from qpack_amd._lib import QPH_Q1
    g = np.load(__file__.replace("test_gpu_kernels.py", "golden/kernels.npz"))
    for key in ("q8_48x1024", "q8_33x896", "q4_48x1024", "q4_33x896"):
        Y = qa.kernel_matmul(g[key + "_q"], g[key + "_s"], g[key + "_X"], order=1)
        np.testing.assert_array_equal(Y, g[key + "_Y"], err_msg=key)
    for key in ("q1_48x1024", "q1_33x896"):   # cols % 128 == 0 (the q1 matrices a model takes)
        Y = qa.kernel_matmul(g[key + "_q"], g[key + "_s"], g[key + "_X"], kind=QPH_Q1, order=1)
        np.testing.assert_array_equal(Y, g[key + "_Y"], err_msg=key)
        y = qa.kernel_matmul(g[key + "_q"], g[key + "_s"], g[key + "_x"][None, :], kind=QPH_Q1, order=1)
        np.testing.assert_array_equal(y[0], g[key + "_y"], err_msg=key + " matvec")
