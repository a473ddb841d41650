"""CPU oracle: restatements of the reference wxx kernels' algorithms.

TEST INFRASTRUCTURE ONLY.  Nothing in ``wxx_amd`` imports this package; only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may use it, and only as the checker (or the timed CPU baseline), never
as the product path.

Each function cites the reference file:line whose behaviour it restates.
The reference itself (WGSL through wgpu-py) cannot run here: wgpu is not
installed, there is no Vulkan ICD, and ``import wxx`` opens a WebGPU device at
import time (reference src/wxx/backend/device.py:258).  The oracle is
therefore pinned against the closed forms of the reference's own tests, the
reference's stated constants, textbook identities and brute force on small
inputs (tests/test_oracle.py), and, for the GEMM, against an exact-order C
restatement of the reference's fp32 fma chain (oracle/csrc/gemm_ref.c).

Modules:
  reductions   sum / mean / sumsq, max / min with the reference tie rule
  activations  softmax, unary activations and their local derivatives
  norms        LayerNorm, RMSNorm, BatchNorm forward and backward
  gemm         batched matmul with bias modes (numpy float64 and C fp32)
  elementwise  broadcast binary ops, scalar ops (pow rules), clamp, equal
"""

from . import activations, elementwise, gemm, norms, reductions

__all__ = ["activations", "elementwise", "gemm", "norms", "reductions"]
