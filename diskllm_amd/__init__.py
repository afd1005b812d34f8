"""MI355X-native implementation of DiskLLM's token-sampling and grammar-mask path.

Layout:
  csrc/hip/   HIP kernels for gfx950 and the batched C ABI (include/diskllm_amd.h)
  csrc/host/  C11 drop-in implementations of include/sampler.h and include/grammar.h
  _lib.py     ctypes binding of the built libdiskllm_amd.so
  api.py      Python host side of the batched path (torch only for device memory/streams)
  workloads.py the synthetic configurations C1-C5
"""
from ._lib import build, lib  # noqa: F401
