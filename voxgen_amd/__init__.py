"""voxgen_amd: the VoxCPM2 BaseLM compute path for one AMD MI355X (gfx950).

The product is libvoxhip.so (C ABI in include/voxhip.h): hand-written HIP
kernels plus the host engine. This package is its Python binding:
  abi      ctypes prototypes of every exported function
  runtime  Context / Buffer / Model handles
  baselm   BaseLmEngine (the reference engine's API)
  gguf     GGUF writer and the C parser's handle
  synth    deterministic synthetic models and inputs
Importing the package does not load the HIP library; the first call does, and
it raises ImportError if libvoxhip.so has not been built (there is no fallback).
"""
from .abi import VxError, load  # noqa: F401

__all__ = ["VxError", "load"]
