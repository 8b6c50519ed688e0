"""pyflamert_amd: MI355X (gfx950) implementation of PyFlameRT's pruned-weight
MatMul/Gemm path.

* ``pyflamert_amd.rocm`` -- numpy/pointer front-end of the C ABI
  (include/pfr_rocm.h): CSR SpMM/SpMV, the Gemm form, 2:4 int8/bf16 GEMM.
* the C++ runtime (InferenceSession / OperatorRegistry / RocmExecutor) lives
  in csrc/runtime and is reached through ``pyflamert_amd.session``.

Nothing here falls back to the CPU: a missing library or device raises.
"""

__version__ = "0.1.0"
