"""CPU checkers for the qpack Llama token loop.  TEST INFRASTRUCTURE, NOT PRODUCT: only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg import this package, and only to check or to time the CPU baseline.

  Oracle    - oracle/liboracle.so, this repository's plain-C restatement of the reference x86 path (oracle.c)
  Ref       - oracle/_ref/libqpref.so, the reference engine compiled from its own sources (oracle/Makefile)
  QpackFile - a numpy reader of QPACK1/QPACK2 files (layout of /root/reference/QPACK2.md:6-12), independent of the product
"""
import ctypes as C
import json
import mmap
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libqpref.so")

OR_Q8, OR_Q4, OR_F32, OR_Q1 = 0, 1, 2, 3


class QpackFile:
    """read-only view of a QPACK1/QPACK2 container: toc, manifest, config and numpy views of the tensors"""

    def __init__(self, path):
        self.f = open(path, "rb")
        self.mm = mmap.mmap(self.f.fileno(), 0, access=mmap.ACCESS_READ)
        if self.mm[:8] not in (b"QPACK1\0\0", b"QPACK2\0\0", b"QPACK3\0\0"):
            raise ValueError(f"not a QPACK1/QPACK2/QPACK3 file: {path}")
        n, _ = struct.unpack("<II", self.mm[8:16])
        self.toc = {}
        for i in range(n):
            b = 16 + 72 * i
            name = self.mm[b:b + 56].rstrip(b"\0").decode()
            off, ln = struct.unpack("<QQ", self.mm[b + 56:b + 72])
            self.toc[name] = (off, ln)
        self.buf = np.frombuffer(self.mm, np.uint8)
        self.decoded = {}
        self.manifest = json.loads(bytes(self.blob("manifest.json")).decode())
        # QPACK3: blobs named in "encoded" hold rANS streams, decoded once here (container.cpp:94-121)
        for name in self.manifest.get("encoded", []):
            self.decoded[name] = rans_decode(self.blob(name))
        self.config = json.loads(bytes(self.blob("config.json")).decode())
        self.tensors = {e["name"]: e for e in self.manifest["tensors"]}

    def blob(self, name):
        if name in self.decoded:
            return self.decoded[name]
        off, ln = self.toc[name]
        return self.buf[off:off + ln]

    def tensor(self, name):
        """(kind, data, scale, rows, cols): q8 int8 [rows, cols] + f32 [rows]; q4 u8 [rows, cols/2] + u16 [rows, cols/32];
        f32 array of the tensor's shape"""
        e = self.tensors[name]
        shape = e["shape"]
        rows, cols = (shape[0], shape[1]) if len(shape) == 2 else (shape[0], 1)
        if e["kind"] == "q8":
            return OR_Q8, self.blob(e["blob"]).view(np.int8).reshape(rows, cols), self.blob(e["scale"]).view(np.float32), rows, cols
        if e["kind"] == "q4":
            return (OR_Q4, self.blob(e["blob"]).reshape(rows, cols // 2), self.blob(e["scale"]).view(np.uint16).reshape(rows, cols // 32),
                    rows, cols)
        if e["kind"] == "q1":
            G = (cols + 127) // 128
            return (OR_Q1, self.blob(e["blob"]).reshape(rows, G * 16), self.blob(e["scale"]).view(np.uint16).reshape(rows, G),
                    rows, cols)
        if e["kind"] == "f32":
            return OR_F32, self.blob(e["blob"]).view(np.float32).reshape(shape), None, rows, cols
        raise ValueError(f"tensor kind {e['kind']} not handled by the oracle")

    def close(self):
        """releases the file; the mapping itself closes once no numpy view of it is alive"""
        self.buf = None
        try:
            self.mm.close()
        except BufferError:
            pass
        self.f.close()


class OrMat(C.Structure):
    _fields_ = [("kind", C.c_int), ("rows", C.c_int), ("cols", C.c_int), ("q", C.c_void_p), ("s", C.c_void_p)]


class OrCfg(C.Structure):
    _fields_ = [("d", C.c_int), ("L", C.c_int), ("nh", C.c_int), ("nkv", C.c_int), ("hd", C.c_int), ("ff", C.c_int),
                ("V", C.c_int), ("ctx", C.c_int), ("tied", C.c_int), ("eps", C.c_float), ("theta", C.c_double)]


class OrLayer(C.Structure):
    _fields_ = [("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p), ("bq", C.c_void_p), ("bk", C.c_void_p), ("bv", C.c_void_p),
                ("wq", OrMat), ("wk", OrMat), ("wv", OrMat), ("wo", OrMat), ("wg", OrMat), ("wu", OrMat), ("wd", OrMat)]


_FP = C.POINTER(C.c_float)
_olib = None


def olib():
    global _olib
    if _olib is None:
        if not os.path.exists(ORACLE_LIB):
            raise ImportError(f"{ORACLE_LIB} is not built (make -C oracle oracle)")
        L = C.CDLL(ORACLE_LIB)
        sig = {
            "or_f32_to_f16": (C.c_uint16, [C.c_float]), "or_f16_to_f32": (C.c_float, [C.c_uint16]),
            "or_quant_act": (None, [_FP, C.c_int, C.c_void_p, _FP]),
            "or_block_sums_q8": (None, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
            "or_group_sums_q4": (None, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
            "or_rows_q8": (None, [C.c_void_p, C.c_void_p, C.c_void_p, _FP, _FP, C.c_int, C.c_int]),
            "or_rows_q4": (None, [C.c_void_p, C.c_void_p, C.c_void_p, _FP, _FP, C.c_int, C.c_int]),
            "or_rows_q1": (None, [C.c_void_p, C.c_void_p, C.c_void_p, _FP, _FP, C.c_int, C.c_int]),
            "or_group_sums_q1": (None, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
            "or_matvec": (None, [C.POINTER(OrMat), _FP, _FP]),
            "or_matmul": (None, [C.POINTER(OrMat), _FP, C.c_int, _FP]),
            "or_rmsnorm": (None, [_FP, _FP, C.c_int, C.c_float, _FP]),
            "or_exp_v": (None, [_FP, _FP, C.c_int]),
            "or_silu_mul": (None, [_FP, _FP, C.c_int]),
            "or_row_f32": (None, [C.POINTER(OrMat), C.c_int, _FP]),
            "or_create": (C.c_void_p, [C.POINTER(OrCfg), C.POINTER(OrMat), C.POINTER(OrMat), C.c_void_p, C.POINTER(OrLayer)]),
            "or_free": (None, [C.c_void_p]), "or_reset": (None, [C.c_void_p]), "or_pos": (C.c_int, [C.c_void_p]),
            "or_set_pos": (C.c_int, [C.c_void_p, C.c_int]),
            "or_step": (C.c_int, [C.c_void_p, C.c_int, C.c_int, _FP]),
            "or_prefill": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, _FP]),
            "or_greedy": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
            "or_kcache": (C.c_void_p, [C.c_void_p]), "or_vcache": (C.c_void_p, [C.c_void_p]),
            "or_set_threads": (None, [C.c_int]),
            "or_set_order": (None, [C.c_int]),
            "or_top_m": (C.c_int, [_FP, C.c_int, C.c_int, C.c_void_p, _FP]),
            "or_rans_raw_size": (C.c_int64, [C.c_void_p, C.c_int64]),
            "or_rans_decode": (C.c_int, [C.c_void_p, C.c_int64, C.c_void_p, C.c_int64]),
            "or_rans_encode": (C.c_int64, [C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_void_p, C.c_int64]),
            "or_rans_freqs": (C.c_int, [C.c_void_p, C.c_int64, C.c_int, C.c_void_p]),
        }
        for k, (r, a) in sig.items():
            getattr(L, k).restype = r
            getattr(L, k).argtypes = a
        _olib = L
    return _olib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _f(a):
    return a.ctypes.data_as(_FP)


def ormat(kind, q, s, rows, cols):
    return OrMat(kind, rows, cols, _p(q), _p(s))


# ------------------------------------------------------------------ kernel-level oracle functions
def quant_act(x):
    x = np.ascontiguousarray(x, np.float32)
    xq = np.empty(len(x), np.int16)
    bs = np.empty((len(x) + 127) // 128, np.float32)
    olib().or_quant_act(_f(x), len(x), _p(xq), _f(bs))
    return xq, bs


def block_sums_q8(q, xq):
    rows, cols = q.shape
    out = np.empty((rows, cols // 128), np.int32)
    olib().or_block_sums_q8(_p(np.ascontiguousarray(q)), rows, cols, _p(xq), _p(out))
    return out


def group_sums_q4(q, xq):
    rows, cols = q.shape[0], q.shape[1] * 2
    out = np.empty((rows, cols // 32), np.int32)
    olib().or_group_sums_q4(_p(np.ascontiguousarray(q)), rows, cols, _p(xq), _p(out))
    return out


def group_sums_q1(q, xq, cols):
    rows, G = q.shape[0], (cols + 127) // 128
    out = np.empty((rows, G), np.int32)
    olib().or_group_sums_q1(_p(np.ascontiguousarray(q)), rows, cols, _p(xq), _p(out))
    return out


def rows_q1(q, s, xq, bs, cols):
    rows = q.shape[0]
    y = np.empty(rows, np.float32)
    olib().or_rows_q1(_p(q), _p(s), _p(xq), _f(bs), _f(y), rows, cols)
    return y


def rows_q8(q, scale, xq, bs):
    rows, cols = q.shape
    y = np.empty(rows, np.float32)
    olib().or_rows_q8(_p(q), _p(scale), _p(xq), _f(bs), _f(y), rows, cols)
    return y


def rows_q4(q, s, xq, bs):
    rows, cols = q.shape[0], q.shape[1] * 2
    y = np.empty(rows, np.float32)
    olib().or_rows_q4(_p(q), _p(s), _p(xq), _f(bs), _f(y), rows, cols)
    return y


def _cols(kind, q):
    return q.shape[1] * {OR_Q4: 2, OR_Q1: 8}.get(kind, 1)


def matvec(kind, q, s, x, cols=None):
    rows = q.shape[0]
    cols = cols or _cols(kind, q)
    m = ormat(kind, q, s, rows, cols)
    y = np.empty(rows, np.float32)
    olib().or_matvec(C.byref(m), _f(np.ascontiguousarray(x, np.float32)), _f(y))
    return y


def matmul(kind, q, s, X, cols=None):
    rows = q.shape[0]
    cols = cols or _cols(kind, q)
    X = np.ascontiguousarray(X, np.float32)
    m = ormat(kind, q, s, rows, cols)
    Y = np.empty((X.shape[0], rows), np.float32)
    olib().or_matmul(C.byref(m), _f(X), X.shape[0], _f(Y))
    return Y


def top_m(x, M):
    """the sampler's M candidates (index, value) in its order (or_top_m)"""
    x = np.ascontiguousarray(x, np.float32)
    idx = np.empty(M, np.int32); val = np.empty(M, np.float32)
    if olib().or_top_m(_f(x), len(x), int(M), _p(idx), _f(val)):
        raise ValueError("top_m: 1 <= M <= len(x) required")
    return idx, val


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    olib().or_rmsnorm(_f(x), _f(np.ascontiguousarray(w, np.float32)), len(x), eps, _f(out))
    return out


def exp_v(x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    olib().or_exp_v(_f(x), _f(y), len(x))
    return y


def silu_mul(g, u):
    g = np.array(g, np.float32)
    olib().or_silu_mul(_f(g), _f(np.ascontiguousarray(u, np.float32)), len(g))
    return g


def f32_to_f16(x):
    return np.array([olib().or_f32_to_f16(float(v)) for v in np.asarray(x, np.float32)], np.uint16)


# ------------------------------------------------------------------ QPACK3 rANS (include/qpack/rans.h, QPACK2.md:30-51)
# the reference's messages (rans.h:53-76, :107-113)
_RANS_ERR = {-1: "rans: truncated", -2: "rans: bad frequency table", -3: "rans: stream overrun", -4: "rans: unknown codec",
             -5: "rans: output capacity", -6: "rans: cannot normalise frequencies", -7: "rans: truncated plane",
             -8: "rans: short blob", -9: "rans: short chunked blob", -10: "rans: truncated chunk table",
             -11: "rans: truncated chunk"}


def rans_raw_size(blob):
    b = np.ascontiguousarray(blob, np.uint8)
    n = olib().or_rans_raw_size(_p(b), len(b))
    if n < 0:
        raise ValueError(_RANS_ERR[n])
    if len(b) and b[0] == 3 and len(b) >= 6:
        n = int(b[2]) | int(b[3]) << 8 | int(b[4]) << 16 | int(b[5]) << 24
    return n


def rans_decode(blob):
    """plain (codec 1 / 2) or chunked (codec 3) blob -> raw bytes (rans.h:101-113)"""
    b = np.ascontiguousarray(blob, np.uint8)
    n = rans_raw_size(b)
    out = np.zeros(max(n, 1), np.uint8)
    e = olib().or_rans_decode(_p(b), len(b), _p(out), n)
    if e:
        raise ValueError(_RANS_ERR[e])
    return out[:n]


def rans_encode(raw, codec, planes):
    """raw bytes -> one plain codec 1 / 2 blob (rans.h:81-93)"""
    r = np.ascontiguousarray(raw, np.uint8)
    cap = 64 + 2 * 256 * 4 + 2 * 2 * len(r) + 64
    out = np.empty(cap, np.uint8)
    n = olib().or_rans_encode(_p(r), len(r), codec, planes, _p(out), cap)
    if n < 0:
        raise ValueError(_RANS_ERR[n])
    return out[:n].copy()


def rans_assemble_chunked(n, chunk_raw, chunks):
    """u8 3 | u8 0 | u32 raw_len | u32 chunk_raw | u32 nchunks | u32 comp_len[nchunks] | chunks (rans.h:115-124)"""
    head = struct.pack("<BBIII", 3, 0, n, chunk_raw, len(chunks)) + b"".join(struct.pack("<I", len(c)) for c in chunks)
    return np.frombuffer(head + b"".join(bytes(c) for c in chunks), np.uint8)


PACK_THRESH, PACK_CHUNK = 32 << 20, 16 << 20   # qpack-pack: blobs above 32 MiB are coded in 16 MiB chunks (:56)


def pack_plan(manifest):
    """blob name -> (codec, planes) of every blob qpack-pack codes, all classes (tools/qpack-pack.cpp:43-53)"""
    plan = {}
    for e in manifest["tensors"]:
        k, b = e["kind"], e["blob"]
        if k == "q4":
            plan[b] = (2, 1); plan[e["scale"]] = (1, 2)
        elif k == "q8":
            plan[b] = (1, 1)
        elif k in ("mxfp4",):
            plan[b] = (1, 1); plan[e["scale"]] = (1, 1)
        elif k in ("q1", "q8g"):
            plan[b] = (1, 1); plan[e["scale"]] = (1, 2)
        elif k == "f16":
            plan[b] = (1, 2)
        elif k == "f32":
            plan[b] = (1, 4)
    return plan


def write_container(path, blobs, magic):
    """blobs: list of (name, bytes) in file order; 64-byte aligned (container.cpp:136-153)"""
    A = 64
    off = (16 + 72 * len(blobs) + A - 1) // A * A
    head = bytearray(magic + struct.pack("<II", len(blobs), 0))
    offs = []
    for name, data in blobs:
        head += name.encode().ljust(56, b"\0") + struct.pack("<QQ", off, len(data))
        offs.append(off)
        off = (off + len(data) + A - 1) // A * A
    with open(path, "wb") as f:
        f.write(head)
        pos = len(head)
        for (name, data), o in zip(blobs, offs):
            f.write(b"\0" * (o - pos))
            f.write(bytes(data))
            pos = o + len(data)


def pack_qpack3(src, dst, threads=8):
    """the qpack-pack transform (tools/qpack-pack.cpp:43-84): every blob of the plan is coded (chunked above 32 MiB) and
    kept coded when that is smaller; the manifest gains "encoded" and "format": "QPACK3"; magic QPACK3"""
    from concurrent.futures import ThreadPoolExecutor
    f = QpackFile(src)
    names = sorted(f.toc, key=lambda n: f.toc[n][0])
    plan = pack_plan(f.manifest)
    jobs = []
    for n in names:
        if n in plan and f.toc[n][1]:
            d = f.blob(n)
            if len(d) > PACK_THRESH:
                jobs += [(n, o, d[o:o + PACK_CHUNK]) for o in range(0, len(d), PACK_CHUNK)]
            else:
                jobs.append((n, 0, d))
    with ThreadPoolExecutor(threads) as ex:
        outs = list(ex.map(lambda j: rans_encode(j[2], *plan[j[0]]), jobs))
    coded = {}
    for (n, o, _), c in zip(jobs, outs):
        coded.setdefault(n, []).append(c)
    man = dict(f.manifest)
    encoded, blobs = [], []
    for n in names:
        d = f.blob(n)
        if n in coded:
            c = coded[n][0] if len(d) <= PACK_THRESH else rans_assemble_chunked(len(d), PACK_CHUNK, coded[n])
            if len(c) < len(d):
                encoded.append(n)
                d = c
        blobs.append([n, d])
    man["encoded"] = encoded
    man["format"] = "QPACK3"
    for b in blobs:
        if b[0] == "manifest.json":
            b[1] = json.dumps(man).encode()
    write_container(dst, blobs, b"QPACK3\0\0")
    f.close()
    return encoded


# ------------------------------------------------------------------ the model
class Oracle:
    """the Llama model of oracle.c over a QPACK file (model_llama.cpp:20-201)"""

    def __init__(self, path, max_ctx=0, threads=0):
        if threads:
            olib().or_set_threads(threads)
        self.file = QpackFile(path)
        c = self.file.config
        d, nh = c["hidden_size"], c["num_attention_heads"]
        self.cfg = OrCfg(d, c["num_hidden_layers"], nh, c["num_key_value_heads"], c.get("head_dim", d // nh), c["intermediate_size"],
                         c["vocab_size"], max_ctx if max_ctx > 0 else min(4096, c.get("max_position_embeddings", 1 << 20)),
                         int(c.get("tie_embeddings", False)), c.get("rms_norm_eps", 1e-6), c.get("rope_theta", 10000.0))
        self._keep = []

        def mat(name):
            k, q, s, r, cc = self.file.tensor(name)
            self._keep.append((q, s))
            return ormat(k, q, s, r, cc)

        def vec(name):
            if name not in self.file.tensors:
                return None
            a = np.ascontiguousarray(self.file.tensor(name)[1], np.float32)
            self._keep.append(a)
            return _p(a)

        self.embed = mat("embed")
        self.head = self.embed if self.cfg.tied else mat("lm_head")
        self.fnorm = vec("final_norm")
        layers = (OrLayer * self.cfg.L)()
        for i in range(self.cfg.L):
            p = f"layers.{i}."
            ly = layers[i]
            ly.attn_norm, ly.ffn_norm = vec(p + "attn_norm"), vec(p + "ffn_norm")
            ly.bq, ly.bk, ly.bv = vec(p + "bq"), vec(p + "bk"), vec(p + "bv")
            ly.wq, ly.wk, ly.wv, ly.wo = mat(p + "wq"), mat(p + "wk"), mat(p + "wv"), mat(p + "wo")
            ly.wg, ly.wu, ly.wd = mat(p + "w_gate"), mat(p + "w_up"), mat(p + "w_down")
        self._layers = layers
        self.m = olib().or_create(C.byref(self.cfg), C.byref(self.embed), C.byref(self.head), self.fnorm, layers)

    def close(self):
        if self.m:
            olib().or_free(self.m)
            self.m = None

    def vocab(self):
        return self.cfg.V

    def pos(self):
        return olib().or_pos(self.m)

    def reset(self):
        olib().or_reset(self.m)

    def set_pos(self, pos):
        if olib().or_set_pos(self.m, int(pos)):
            raise RuntimeError("oracle set_pos: out of range")

    def step(self, tok, want=1):
        out = np.empty(self.cfg.V if want == 1 else self.cfg.d, np.float32) if want else None
        if olib().or_step(self.m, int(tok), want, _f(out) if out is not None else None):
            raise RuntimeError("oracle step: token out of range or context full")
        return out

    def prefill(self, toks, want=1):
        toks = np.ascontiguousarray(toks, np.int32)
        out = np.empty(self.cfg.V if want == 1 else self.cfg.d, np.float32) if want else None
        if olib().or_prefill(self.m, _p(toks), len(toks), want, _f(out) if out is not None else None):
            raise RuntimeError("oracle prefill: token out of range or context full")
        return out

    def greedy_run(self, tok, n):
        out = np.empty(n, np.int32)
        if olib().or_greedy(self.m, int(tok), n, _p(out)) < 0:
            raise RuntimeError("oracle greedy: context full")
        return out

    def kv_cache(self):
        n = self.cfg.L * self.cfg.ctx * self.cfg.nkv * self.cfg.hd
        k = np.ctypeslib.as_array(C.cast(olib().or_kcache(self.m), C.POINTER(C.c_uint16)), (n,))
        v = np.ctypeslib.as_array(C.cast(olib().or_vcache(self.m), C.POINTER(C.c_uint16)), (n,))
        shape = (self.cfg.L, self.cfg.ctx, self.cfg.nkv * self.cfg.hd)
        return k.reshape(shape), v.reshape(shape)


# ------------------------------------------------------------------ the compiled reference
_rlib = None


def ref_available():
    return os.path.exists(REF_LIB)


def rlib(threads=0):
    """the reference engine; `threads` must be given on the first call (qp::set_threads before the pool exists)"""
    global _rlib
    if _rlib is None:
        if not os.path.exists(REF_LIB):
            raise ImportError(f"{REF_LIB} is not built (make -C oracle ref, needs /root/reference)")
        L = C.CDLL(REF_LIB)
        P, I = C.c_void_p, C.c_int
        sig = {
            "qpref_error": (C.c_char_p, []), "qpref_set_threads": (None, [I]), "qpref_threads": (I, []),
            "qpref_load": (I, [C.c_char_p, I, C.POINTER(P)]), "qpref_free": (None, [P]),
            "qpref_vocab": (I, [P]), "qpref_hidden": (I, [P]), "qpref_pos": (I, [P]), "qpref_max_ctx": (I, [P]),
            "qpref_reset": (None, [P]),
            "qpref_step": (I, [P, I, I, _FP]), "qpref_prefill": (I, [P, P, I, I, _FP]), "qpref_greedy": (I, [P, I, I, P]),
            "qpref_snapshot": (C.c_int64, [P, P, C.c_int64]), "qpref_restore": (I, [P, P, C.c_int64]),
            "qpref_matvec": (I, [I, P, P, I, I, _FP, _FP]), "qpref_matmul": (I, [I, P, P, I, I, _FP, I, _FP, I]),
            "qpref_rows_q8": (None, [P, P, P, _FP, _FP, I, I]), "qpref_rows_q4": (None, [P, P, P, _FP, _FP, I, I]),
            "qpref_rows_q1": (None, [P, P, P, _FP, _FP, I, I]),
            "qpref_rmsnorm": (None, [_FP, _FP, I, C.c_float, _FP]), "qpref_silu_mul": (None, [_FP, _FP, I]),
            "qpref_exp_v": (None, [_FP, _FP, I]), "qpref_to_f16": (None, [_FP, P, I]),
            "qpref_row_f32": (None, [I, P, P, I, I, I, _FP]),
            "qpref_rans_encode": (I, [P, C.c_int64, I, I, P, C.c_int64, C.POINTER(C.c_int64)]),
            "qpref_rans_decode": (I, [P, C.c_int64, P]),
            "qpref_prefill_all": (I, [P, P, I, _FP, I]), "qpref_rewind": (I, [P, I]), "qpref_sampler_topk": (I, [_FP, I, I, P]), "qpref_rans_raw_size": (C.c_int64, [P, C.c_int64]),
        }
        for k, (r, a) in sig.items():
            getattr(L, k).restype = r
            getattr(L, k).argtypes = a
        if threads:
            L.qpref_set_threads(threads)
        _rlib = L
    return _rlib


class Ref:
    """qp::load_model on the compiled reference (CPU)"""

    def __init__(self, path, max_ctx=0, threads=0):
        L = rlib(threads)
        h = C.c_void_p()
        if L.qpref_load(str(path).encode(), max_ctx, C.byref(h)):
            raise RuntimeError(L.qpref_error().decode())
        self.L, self.m = L, h

    def _ck(self, st):
        if st:
            raise RuntimeError(self.L.qpref_error().decode())

    def close(self):
        if self.m:
            self.L.qpref_free(self.m)
            self.m = None

    def vocab(self):
        return self.L.qpref_vocab(self.m)

    def hidden(self):
        return self.L.qpref_hidden(self.m)

    def pos(self):
        return self.L.qpref_pos(self.m)

    def reset(self):
        self.L.qpref_reset(self.m)

    def step(self, tok, want=1):
        out = np.empty(self.vocab() if want == 1 else self.hidden(), np.float32) if want else None
        self._ck(self.L.qpref_step(self.m, int(tok), want, _f(out) if out is not None else None))
        return out

    def prefill(self, toks, want=1):
        toks = np.ascontiguousarray(toks, np.int32)
        out = np.empty(self.vocab() if want == 1 else self.hidden(), np.float32) if want else None
        self._ck(self.L.qpref_prefill(self.m, _p(toks), len(toks), want, _f(out) if out is not None else None))
        return out

    def greedy_run(self, tok, n):
        out = np.empty(n, np.int32)
        self._ck(self.L.qpref_greedy(self.m, int(tok), n, _p(out)))
        return out

    def rewind(self, pos):
        return bool(self.L.qpref_rewind(self.m, int(pos)))

    def prefill_all(self, toks, exact=True):
        """Model::prefill_all: the logits of every position [n, vocab]; under ExactBatches when exact"""
        toks = np.ascontiguousarray(toks, np.int32)
        out = np.empty((len(toks), self.vocab()), np.float32)
        self._ck(self.L.qpref_prefill_all(self.m, _p(toks), len(toks), _f(out), int(exact)))
        return out

    def snapshot(self):
        n = self.L.qpref_snapshot(self.m, None, 0)
        buf = np.empty(n, np.uint8)
        if self.L.qpref_snapshot(self.m, _p(buf), n) != n:
            raise RuntimeError(self.L.qpref_error().decode())
        return buf.tobytes()

    def restore(self, s):
        buf = np.frombuffer(s, np.uint8)
        self._ck(self.L.qpref_restore(self.m, _p(buf), len(buf)))


def ref_sampler_topk(x, M):
    """the indices of the reference sampler's top-M candidates (Sampler::dist with top_k = M and no other filter), in its
    order: the compiled reference's top_m + sort (/root/reference/src/sampler.cpp:12-27, :41-42)"""
    L = rlib()
    x = np.ascontiguousarray(x, np.float32)
    idx = np.empty(M, np.int32)
    if L.qpref_sampler_topk(_f(x), len(x), int(M), _p(idx)):
        raise RuntimeError(L.qpref_error().decode())
    return idx
