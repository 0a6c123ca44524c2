"""Seeded synthetic Llama-family QPACK2 files (random init; rules in csrc/host/synth.cpp) and the benchmark configurations.

The five benchmark configurations: C1 Qwen2.5-0.5B q8, C2 the same in q4 (embed / head q8), C3
Llama-3-8B q8, C4 the same model for prefill, C5 Qwen2.5-7B q4m.  MINI is a small shape for CPU-side oracle checks.
"""
import ctypes as C
from dataclasses import dataclass

from ._lib import SynthSpecC, check, lib


@dataclass
class Shape:
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    tied: bool
    qkv_bias: bool
    rope_theta: float
    model_type: str
    rms_eps: float = 1e-6
    max_pos: int = 32768
    q4: bool = False
    q4m_alt: bool = False
    more_bits: bool = False
    q4_head: bool = False
    mlp_q1: bool = False


QWEN05 = dict(hidden=896, layers=24, heads=14, kv_heads=2, head_dim=64, ffn=4864, vocab=151936, tied=True, qkv_bias=True,
              rope_theta=1e6, model_type="qwen2")
LLAMA8 = dict(hidden=4096, layers=32, heads=32, kv_heads=8, head_dim=128, ffn=14336, vocab=128256, tied=False, qkv_bias=False,
              rope_theta=5e5, model_type="llama", rms_eps=1e-5)
QWEN7 = dict(hidden=3584, layers=28, heads=28, kv_heads=4, head_dim=128, ffn=18944, vocab=152064, tied=False, qkv_bias=True,
             rope_theta=1e6, model_type="qwen2")

CONFIGS = {
    "c1": Shape(**QWEN05),
    "c2": Shape(**QWEN05, q4=True),
    "c3": Shape(**LLAMA8),
    "c4": Shape(**LLAMA8),
    "c5": Shape(**QWEN7, q4=True, q4m_alt=True),
    # small shapes (oracle-speed) with the same structure: GQA, bias, tied / untied, q8 / q4 / q4m
    "mini": Shape(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=1000, tied=True, qkv_bias=True,
                  rope_theta=1e6, model_type="qwen2"),
    "mini128": Shape(hidden=512, layers=2, heads=4, kv_heads=1, head_dim=128, ffn=768, vocab=2048, tied=False, qkv_bias=False,
                     rope_theta=5e5, model_type="llama", rms_eps=1e-5),
    "mini_q4": Shape(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=1000, tied=True, qkv_bias=True,
                     rope_theta=1e6, model_type="qwen2", q4=True),
    "mini_q4m": Shape(hidden=384, layers=3, heads=6, kv_heads=2, head_dim=64, ffn=640, vocab=1500, tied=False, qkv_bias=True,
                      rope_theta=1e6, model_type="qwen2", q4=True, q4m_alt=True),
    # k / v row counts that end inside a 128-row product tile (192 and 64 rows): the prompt's segmented q / k / v launch
    "mini_odd": Shape(hidden=256, layers=2, heads=6, kv_heads=3, head_dim=64, ffn=384, vocab=900, tied=False, qkv_bias=True,
                      rope_theta=1e6, model_type="qwen2"),
    "mini_odd_q4": Shape(hidden=256, layers=2, heads=2, kv_heads=1, head_dim=64, ffn=384, vocab=900, tied=True,
                         qkv_bias=True, rope_theta=1e6, model_type="qwen2", q4=True),
    # seven query heads per kv group, as C1 (head dim 64) and C5 (head dim 128) have them
    "mini_r7": Shape(hidden=256, layers=2, heads=14, kv_heads=2, head_dim=64, ffn=512, vocab=1000, tied=True,
                     qkv_bias=True, rope_theta=1e6, model_type="qwen2"),
    "mini_r7h": Shape(hidden=256, layers=2, heads=7, kv_heads=1, head_dim=128, ffn=512, vocab=1000, tied=False,
                      qkv_bias=True, rope_theta=1e6, model_type="qwen2", q4=True, q4m_alt=True),
    # qpack-quantize's other outputs: q1 MLP matrices (q1m keeps the more_bits downs in q8), the real q4m layer policy,
    # and q4 with a q4 embedding / head
    "mini_q1": Shape(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=1000, tied=True, qkv_bias=True,
                     rope_theta=1e6, model_type="qwen2", mlp_q1=True),
    "mini_q1m": Shape(hidden=384, layers=9, heads=6, kv_heads=2, head_dim=64, ffn=640, vocab=1500, tied=False, qkv_bias=True,
                      rope_theta=1e6, model_type="qwen2", mlp_q1=True, more_bits=True),
    "mini_q4mb": Shape(hidden=384, layers=9, heads=6, kv_heads=2, head_dim=64, ffn=640, vocab=1500, tied=False, qkv_bias=True,
                       rope_theta=1e6, model_type="qwen2", q4=True, more_bits=True),
    "mini_q4h": Shape(hidden=512, layers=2, heads=4, kv_heads=1, head_dim=128, ffn=768, vocab=2048, tied=False, qkv_bias=False,
                      rope_theta=5e5, model_type="llama", rms_eps=1e-5, q4=True, q4_head=True),
    # the 8B shape with 1-bit MLP matrices (q1, attention q8): a decode workload for the q1 matvec
    "c3_q1": Shape(**LLAMA8, mlp_q1=True),
}


def write_synthetic(shape, path, seed=1234, std=0.02, threads=0):
    """write a QPACK2 file of `shape` (a Shape or a CONFIGS key) with N(0, std) weights from `seed`"""
    if isinstance(shape, str):
        shape = CONFIGS[shape]
    s = SynthSpecC()
    for f in ("hidden", "layers", "heads", "kv_heads", "head_dim", "ffn", "vocab", "max_pos"):
        setattr(s, f, int(getattr(shape, f)))
    s.tied, s.qkv_bias, s.q4, s.q4m_alt = int(shape.tied), int(shape.qkv_bias), int(shape.q4), int(shape.q4m_alt)
    s.more_bits, s.q4_head, s.mlp_q1 = int(shape.more_bits), int(shape.q4_head), int(shape.mlp_q1)
    s.rms_eps, s.rope_theta, s.std, s.seed = shape.rms_eps, shape.rope_theta, std, seed
    s.model_type = shape.model_type.encode()[:31]
    check(lib().qph_synth_write(C.byref(s), str(path).encode(), int(threads)))
    return str(path)


def kv_fill_snapshot(shape, T, seed):
    """a snapshot in the reference's layout (/root/reference/src/model_llama.cpp:55-63: int32 position, then per layer the
    K rows and the V rows of positions [0, T)) whose fp16 values are N(0, 1) from `seed`: how the C5 workload fills its
    16K context"""
    import numpy as np
    if isinstance(shape, str):
        shape = CONFIGS[shape]
    kvd = shape.kv_heads * shape.head_dim
    rng = np.random.default_rng(seed)
    parts = [np.int32(T).tobytes()]
    for _ in range(shape.layers):
        for _ in range(2):
            parts.append(rng.standard_normal((T, kvd), dtype=np.float32).astype(np.float16).tobytes())
    return b"".join(parts)
