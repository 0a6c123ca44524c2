"""qpack_amd: the MI355X (gfx950) Llama-family token loop of qpack behind a C ABI.

  HipLlama.load(path)   - a QPACK1/QPACK2 file on the GPU (the qp::Model surface: step / prefill / greedy_run / ...)
  write_synthetic(...)  - seeded random-init QPACK2 models of the benchmark shapes (C1-C5)
  kernel_matvec(...)    - the product's matvec kernel on one matrix, with its exact int32 accumulators (parity hook)
  kernel_matmul(...)    - the product's batched prefill kernels on one q8 / q4 matrix (parity hook)
  kernel_topk(...)      - the device top-M selection of step_topk on one vector (parity hook)
"""
from ._lib import LIB_PATH, QPH_F32, QPH_Q1, QPH_Q4, QPH_Q8, QphError, device_count, lib
from .model import HipLlama, kernel_matmul, kernel_matvec, kernel_rans_decode, kernel_topk, pack, time_copy
from .synth import CONFIGS, Shape, kv_fill_snapshot, write_synthetic

__all__ = ["HipLlama", "kernel_matmul", "kernel_matvec", "kernel_rans_decode", "kernel_topk", "pack", "time_copy", "write_synthetic", "kv_fill_snapshot", "CONFIGS", "Shape", "QphError", "device_count", "lib", "LIB_PATH",
           "QPH_F32", "QPH_Q8", "QPH_Q4", "QPH_Q1"]
