"""HipLlama: the Python face of the C ABI, method for method the reference's qp::Model
(/root/reference/include/qpack/qpack.h:128-171).  Used by the tests and bench.py; C++ callers use include/qpack_hip.h
directly."""
import ctypes as C

import numpy as np

from ._lib import Config, LoadStatsC, check, lib


def _fptr(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _iptr(a):
    return a.ctypes.data_as(C.POINTER(C.c_int))


class HipLlama:
    def __init__(self, handle):
        self._h = C.c_void_p(handle)
        cfg = Config()
        check(lib().qph_config_of(self._h, C.byref(cfg)))
        self.config = cfg

    @classmethod
    def load(cls, path, max_ctx=0):
        """load_model(path, max_ctx) with QPACK_DEVICE selecting this backend (model_llama.cpp:221-235)"""
        h = C.c_void_p()
        check(lib().qph_load(str(path).encode(), int(max_ctx), C.byref(h)))
        return cls(h.value)

    def close(self):
        if self._h:
            lib().qph_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # ---- queries (qpack.h:131-134)
    def vocab(self):
        return lib().qph_vocab(self._h)

    def hidden(self):
        return lib().qph_hidden(self._h)

    def max_ctx(self):
        return lib().qph_max_ctx(self._h)

    def pos(self):
        return lib().qph_pos(self._h)

    # ---- token loop
    def step(self, token, want=1):
        """Model::step: want 0 -> None, 1 -> logits [vocab] float32, 2 -> final normed hidden [hidden]"""
        out = None
        if want == 1:
            out = np.empty(self.vocab(), np.float32)
        elif want == 2:
            out = np.empty(self.hidden(), np.float32)
        check(lib().qph_step(self._h, int(token), int(want), _fptr(out) if out is not None else None))
        return out

    def prefill(self, tokens, want=1):
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        out = None
        if want == 1:
            out = np.empty(self.vocab(), np.float32)
        elif want == 2:
            out = np.empty(self.hidden(), np.float32)
        check(lib().qph_prefill(self._h, _iptr(toks), len(toks), int(want), _fptr(out) if out is not None else None))
        return out

    def greedy_run(self, token, n):
        out = np.zeros(max(n, 1), np.int32)
        got = C.c_int(0)
        check(lib().qph_greedy_run(self._h, int(token), int(n), _iptr(out), C.byref(got)))
        return out[:got.value]

    def prefill_all(self, tokens):
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((len(toks), self.vocab()), np.float32)
        check(lib().qph_prefill_all(self._h, _iptr(toks), len(toks), _fptr(out)))
        return out

    def step_topk(self, token, M):
        """step with the logits kept on the device: their M largest (index, value) pairs, value descending and the
        lower index first among equal values (the sampler's top_m order, sampler.cpp:12-27)"""
        idx = np.empty(M, np.int32); val = np.empty(M, np.float32)
        check(lib().qph_step_topk(self._h, int(token), int(M), _iptr(idx), _fptr(val)))
        return idx, val

    def prefill_topk(self, tokens, M):
        """prefill with the last token's logits kept on the device: their M largest (index, value) pairs"""
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        idx = np.empty(M, np.int32); val = np.empty(M, np.float32)
        check(lib().qph_prefill_topk(self._h, _iptr(toks), len(toks), int(M), _iptr(idx), _fptr(val)))
        return idx, val

    def reset(self):
        check(lib().qph_reset(self._h))

    def set_order(self, mode):
        """0: this library's kernels (default); 1: the reference CPU path's arithmetic order everywhere (bit-identical
        logits and greedy streams; slower)"""
        check(lib().qph_set_order(self._h, int(mode)))

    def rewind(self, pos):
        ok = C.c_int(0)
        check(lib().qph_rewind(self._h, int(pos), C.byref(ok)))
        return bool(ok.value)

    def checkpoint(self):
        return np.int32(self.pos()).tobytes()

    def rollback(self, c):
        check(lib().qph_set_pos(self._h, int(np.frombuffer(c, np.int32)[0])))

    def snapshot(self):
        n = C.c_int64(0)
        check(lib().qph_snapshot_size(self._h, C.byref(n)))
        buf = np.empty(n.value, np.uint8)
        check(lib().qph_snapshot(self._h, buf.ctypes.data_as(C.c_void_p), n.value))
        return buf.tobytes()

    def restore(self, s):
        buf = np.frombuffer(s, np.uint8)
        check(lib().qph_restore(self._h, buf.ctypes.data_as(C.c_void_p), len(buf)))

    # ---- measurement
    def load_stats(self):
        """the QPACK3 decode of this model's load: planes, coded / raw bytes, upload / decode / both ms (the decode
        launches run under the upload, one per upload round), rounds"""
        st = LoadStatsC()
        check(lib().qph_load_stats_of(self._h, C.byref(st)))
        return {"planes": st.planes, "coded_bytes": st.coded_bytes, "raw_bytes": st.raw_bytes, "upload_ms": st.upload_ms,
                "decode_ms": st.decode_ms, "total_ms": st.total_ms, "rounds": st.rounds}

    def time_greedy(self, token, n):
        ms = C.c_float(0)
        check(lib().qph_time_greedy(self._h, int(token), int(n), C.byref(ms)))
        return ms.value

    def time_kernel(self, which, iters):
        ms, b = C.c_float(0), C.c_double(0)
        check(lib().qph_time_kernel(self._h, int(which), int(iters), C.byref(ms), C.byref(b)))
        return ms.value, b.value


def time_copy(nbytes, iters=4):
    """mean duration (ms) of the library's plain device copy kernel k_copy over nbytes (qph_time_copy)"""
    ms = C.c_float()
    check(lib().qph_time_copy(int(nbytes), int(iters), C.byref(ms)))
    return ms.value


def kernel_matvec(kind, q, scale, x):
    """the product's matvec kernel on one matrix: returns (y, exact int32 sums, int16 activation, block scales)"""
    from ._lib import QPH_Q1, QPH_Q4
    q = np.ascontiguousarray(q)
    scale = np.ascontiguousarray(scale)
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows = q.shape[0]
    cols = q.shape[1] * {QPH_Q4: 2, QPH_Q1: 8}.get(kind, 1)
    y = np.empty(rows, np.float32)
    sums = np.empty((rows, cols // 32 if kind == QPH_Q4 else cols // 128), np.int32)
    xq = np.empty(cols, np.int16)
    bs = np.empty(cols // 128, np.float32)
    check(lib().qph_kernel_matvec(kind, q.ctypes.data_as(C.c_void_p), scale.ctypes.data_as(C.c_void_p), rows, cols, _fptr(x),
                                  _fptr(y), sums.ctypes.data_as(C.POINTER(C.c_int32)), xq.ctypes.data_as(C.POINTER(C.c_int16)),
                                  _fptr(bs)))
    return y, sums, xq, bs


def kernel_matmul(q, scale, X, kind=None, order=0):
    """the product's batched prefill kernels on one matrix: Y[B, rows] = X[B, cols] W^T (qph_kernel_matmul); q8 (int8
    q, f32 scale) or q4 (packed u8 q, fp16-bits scale per 32 columns); order=1: the reference-order products
    (qph_kernel_matmul_ref), which also take kind=QPH_Q1 (sign bits [rows][cols / 8], fp16-bits scale per 128 columns)"""
    from ._lib import QPH_Q1, QPH_Q4, QPH_Q8
    if kind is None:
        kind = QPH_Q8 if q.dtype == np.int8 else QPH_Q4
    q = np.ascontiguousarray(q)
    scale = np.ascontiguousarray(scale)
    X = np.ascontiguousarray(X, dtype=np.float32)
    rows = q.shape[0]
    cols = q.shape[1] if kind == QPH_Q8 else 2 * q.shape[1] if kind == QPH_Q4 else 8 * q.shape[1]
    B = X.shape[0]
    assert X.shape[1] == cols
    Y = np.empty((B, rows), np.float32)
    f = lib().qph_kernel_matmul_ref if order else lib().qph_kernel_matmul
    check(f(kind, q.ctypes.data_as(C.c_void_p), scale.ctypes.data_as(C.c_void_p), rows, cols, _fptr(X), B, _fptr(Y)))
    return Y


def kernel_topk(x, M):
    """the device top-M selection on a host vector (qph_kernel_topk): (idx, val) of the M largest, value descending,
    lower index first among equal values"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    idx = np.empty(M, np.int32); val = np.empty(M, np.float32)
    check(lib().qph_kernel_topk(_fptr(x), len(x), int(M), _iptr(idx), _fptr(val)))
    return idx, val


def kernel_rans_decode(blob):
    """rans::decode of one QPACK3 blob on the GPU (qph_kernel_rans_decode): (raw bytes, decode-kernel ms)"""
    b = np.ascontiguousarray(np.frombuffer(bytes(blob), np.uint8) if not isinstance(blob, np.ndarray) else blob, np.uint8)
    raw = C.c_int64(0)
    if len(b) >= 6:
        raw.value = int(b[2]) | int(b[3]) << 8 | int(b[4]) << 16 | int(b[5]) << 24
    out = np.empty(max(raw.value, 1), np.uint8)
    ms = C.c_float(0)
    check(lib().qph_kernel_rans_decode(b.ctypes.data, len(b), out.ctypes.data, len(out), C.byref(raw), C.byref(ms)))
    return out[:raw.value], ms.value


def pack(src, dst, threads=8):
    """qpack-pack src dst (qph_pack): QPACK2 -> QPACK3; returns the number of coded blobs"""
    n = C.c_int(0)
    check(lib().qph_pack(str(src).encode(), str(dst).encode(), int(threads), C.byref(n)))
    return n.value
