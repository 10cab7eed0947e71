"""KernRelay-MI355X: the single-GPU relay path (row-tiled producer GEMM ->
flag-released consumers) as hand-written HIP kernels for gfx950 behind the
reference's C ABI (include/kernrelay.h).

Modules
  libapi    ctypes wrapper of the six ABI entry points (reference libapi.py)
  ops       op-level kernel bindings on torch device tensors
  schedule  DAG model and fixed row-split schedules for kr_plan_run
  modeldir  synthetic model directories in the reference's export format
  build     compiles libkernrelay.so for gfx950
"""

__version__ = "0.1.0"
