"""qph_topk_noalloc, the allocation-free entry point: the top-M of device buffers with its scratch in a fixed per-GPU
device array, against qph_kernel_topk (the allocating entry point it varies) on the same inputs - indices and values
bit-identical - on two calls in a row, the second with a smaller input, so a stale first call's keys in the shared
array would show.  Device buffers come from the HIP runtime the library itself uses (hipMalloc through ctypes): the
test allocates, the entry point does not."""
import ctypes as C

import numpy as np
import pytest

import qpack_amd as qa
from qpack_amd._lib import lib

pytestmark = pytest.mark.gpu


def hip():
    lib()   # the library's own libamdhip64 is loaded first; this opens the same instance
    H = C.CDLL("libamdhip64.so.7")
    H.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    H.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    H.hipFree.argtypes = [C.c_void_p]
    return H


def test_topk_noalloc_matches_allocating_entry_point():
    H = hip()
    bufs = []

    def dalloc(n):
        p = C.c_void_p()
        assert H.hipMalloc(C.byref(p), n) == 0
        bufs.append(p)
        return p
    try:
        rng = np.random.default_rng(17)
        for n, M in ((151936, 512), (20000, 40)):   # second call smaller: a stale key from the first would win
            print(f"topk_noalloc n={n} M={M}", flush=True)
            x = (rng.standard_normal(n) * 3).astype(np.float32)
            x[::97] = np.round(x[::97])             # ties: the lower index must come first
            dx, di, dv = dalloc(4 * n), dalloc(4 * M), dalloc(4 * M)
            assert H.hipMemcpy(dx, x.ctypes.data, 4 * n, 1) == 0
            qa._lib.check(lib().qph_topk_noalloc(dx, n, M, di, dv, None))
            assert H.hipDeviceSynchronize() == 0
            idx = np.empty(M, np.int32); val = np.empty(M, np.float32)
            assert H.hipMemcpy(idx.ctypes.data, di, 4 * M, 2) == 0
            assert H.hipMemcpy(val.ctypes.data, dv, 4 * M, 2) == 0
            ei, ev = qa.kernel_topk(x, M)
            np.testing.assert_array_equal(idx, ei)
            np.testing.assert_array_equal(val, ev)
        with pytest.raises(qa.QphError, match="262144"):
            qa._lib.check(lib().qph_topk_noalloc(bufs[0], 262145, 4, bufs[1], bufs[2], None))
    finally:
        for p in bufs:
            H.hipFree(p)
