"""ctypes binding of libqpack_hip.so (the C ABI declared in include/qpack_hip.h).

The library is built in-tree by qpack_amd/csrc/Makefile (driven by __graft_entry__.build()).  Loading fails loudly when it is missing: there is no CPU fallback
on the product path.
"""
import ctypes as C
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libqpack_hip.so")

QPH_F32, QPH_Q8, QPH_Q4, QPH_Q1 = 0, 1, 2, 3


class QphError(RuntimeError):
    """an error reported by the C ABI (status -1 + qph_last_error), the analogue of the reference's std::runtime_error"""


class Config(C.Structure):
    _fields_ = [("hidden", C.c_int), ("layers", C.c_int), ("heads", C.c_int), ("kv_heads", C.c_int), ("head_dim", C.c_int),
                ("ffn", C.c_int), ("vocab", C.c_int), ("tied", C.c_int), ("qkv_bias", C.c_int), ("max_pos", C.c_int),
                ("rms_eps", C.c_float), ("rope_theta", C.c_double)]


class Tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("kind", C.c_int), ("rows", C.c_int64), ("cols", C.c_int64),
                ("data", C.c_void_p), ("scale", C.c_void_p), ("data_coded", C.c_int64), ("scale_coded", C.c_int64)]


class LoadStatsC(C.Structure):
    _fields_ = [("planes", C.c_int), ("coded_bytes", C.c_int64), ("raw_bytes", C.c_int64), ("upload_ms", C.c_float),
                ("decode_ms", C.c_float), ("total_ms", C.c_float), ("rounds", C.c_int)]


class SynthSpecC(C.Structure):
    _fields_ = [("hidden", C.c_int), ("layers", C.c_int), ("heads", C.c_int), ("kv_heads", C.c_int), ("head_dim", C.c_int),
                ("ffn", C.c_int), ("vocab", C.c_int), ("tied", C.c_int), ("qkv_bias", C.c_int), ("max_pos", C.c_int),
                ("q4", C.c_int), ("q4m_alt", C.c_int), ("rms_eps", C.c_float), ("rope_theta", C.c_double), ("std", C.c_float),
                ("seed", C.c_uint64), ("model_type", C.c_char * 32), ("more_bits", C.c_int), ("q4_head", C.c_int),
                ("mlp_q1", C.c_int)]


_P = C.c_void_p
_I = C.c_int
_FP = C.POINTER(C.c_float)
_IP = C.POINTER(C.c_int)

# name: (restype, argtypes) for every symbol of include/qpack_hip.h
SIGNATURES = {
    "qph_last_error": (C.c_char_p, []),
    "qph_device_count": (_I, [_IP]),
    "qph_create": (_I, [C.POINTER(Config), C.POINTER(Tensor), _I, _I, C.POINTER(_P)]),
    "qph_load": (_I, [C.c_char_p, _I, C.POINTER(_P)]),
    "qph_destroy": (None, [_P]),
    "qph_vocab": (_I, [_P]),
    "qph_hidden": (_I, [_P]),
    "qph_max_ctx": (_I, [_P]),
    "qph_pos": (_I, [_P]),
    "qph_config_of": (_I, [_P, C.POINTER(Config)]),
    "qph_step": (_I, [_P, _I, _I, _FP]),
    "qph_prefill": (_I, [_P, _IP, _I, _I, _FP]),
    "qph_greedy_run": (_I, [_P, _I, _I, _IP, _IP]),
    "qph_prefill_all": (_I, [_P, _IP, _I, _FP]),
    "qph_step_topk": (_I, [_P, _I, _I, _IP, _FP]),
    "qph_prefill_topk": (_I, [_P, _IP, _I, _I, _IP, _FP]),
    "qph_reset": (_I, [_P]),
    "qph_rewind": (_I, [_P, _I, _IP]),
    "qph_set_pos": (_I, [_P, _I]),
    "qph_snapshot_size": (_I, [_P, C.POINTER(C.c_int64)]),
    "qph_snapshot": (_I, [_P, C.c_void_p, C.c_int64]),
    "qph_restore": (_I, [_P, C.c_void_p, C.c_int64]),
    "qph_set_order": (_I, [_P, _I]),
    "qph_time_greedy": (_I, [_P, _I, _I, _FP]),
    "qph_time_kernel": (_I, [_P, _I, _I, _FP, C.POINTER(C.c_double)]),
    "qph_time_copy": (_I, [C.c_int64, _I, _FP]),
    "qph_kernel_matvec": (_I, [_I, _P, _P, _I, _I, _FP, _FP, C.POINTER(C.c_int32), C.POINTER(C.c_int16), _FP]),
    "qph_kernel_matmul": (_I, [_I, _P, _P, _I, _I, _FP, _I, _FP]),
    "qph_kernel_matmul_ref": (_I, [_I, _P, _P, _I, _I, _FP, _I, _FP]),
    "qph_kernel_topk": (_I, [_FP, _I, _I, _IP, _FP]),
    "qph_topk_noalloc": (_I, [_P, _I, _I, _P, _P, _P]),
    "qph_synth_write": (_I, [C.POINTER(SynthSpecC), C.c_char_p, _I]),
    "qph_load_stats_of": (_I, [C.c_void_p, C.POINTER(LoadStatsC)]),
    "qph_kernel_rans_decode": (_I, [C.c_void_p, C.c_int64, C.c_void_p, C.c_int64, C.POINTER(C.c_int64), _FP]),
    "qph_pack": (_I, [C.c_char_p, C.c_char_p, _I, _IP]),
}

_lib = None


def lib():
    """the loaded library; raises a clear error when it has not been built"""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
                              "(the HIP path has no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(status):
    if status != 0:
        raise QphError(lib().qph_last_error().decode(errors="replace"))


def device_count():
    n = C.c_int(0)
    check(lib().qph_device_count(C.byref(n)))
    return n.value
