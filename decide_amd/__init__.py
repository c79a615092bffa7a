"""decide_amd — MI355X-native (gfx950) prefill GEMM path of decide.

The product is the HIP library ``libdecide_hip.so`` (C ABI in
``include/decide_hip.h``, sources in ``decide_amd/csrc``). This package is
its Python face: ``kernels`` mirrors decide-engine's kernel wrappers
(``Gemm``, ``Head``, ``Norm``) over the C ABI, ``synth`` makes the seeded
inputs. Nothing here computes on the CPU in place of the library.
"""

from . import _lib, synth  # noqa: F401
from .kernels import Context, Epilogue, Gemm, GemmImpl, Head, Kernels, Norm  # noqa: F401

__all__ = ["Context", "Epilogue", "Gemm", "GemmImpl", "Head", "Kernels", "Norm", "synth"]
