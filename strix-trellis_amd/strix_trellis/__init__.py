"""strix_trellis for MI355X: EXL3 / QTIP trellis linear layers on gfx950.

The compute path is libstrix_trellis.so (hand-written HIP for gfx950 behind
the reference's C ABI v1, include/strix_trellis.h).  This package is the thin
Python host layer over it:

``abi``      ctypes mirror of the C ABI (descriptors, statuses, library loader);
``runtime``  contexts, prepared weights, GEMV/GEMM calls, plans (on torch tensors or
             ``device`` arrays);
``device``   device memory and streams from the HIP runtime (ctypes), for hosts without torch;
``loader``   EXL3 groups mapped from local safetensors files, their transport, and
             ``Exl3Tensor.matmul(x, production=True)`` on the GPU (NumPy in and out);
``tp``       two-rank tensor-parallel views of EXL3 groups (rank_partition);
``fixture``  the STGPU001 fixture container (reader and writer) and the manifest
             fixtures of EXL3 groups (``load_fixture``).
"""
from . import abi
from .abi import StrixError
from .fixture import load_fixture
from .loader import Exl3Tensor, SafetensorsFile, decode_legacy_signs, load_exl3
from .tp import rank_partition

__all__ = ["abi", "StrixError", "Exl3Tensor", "SafetensorsFile", "decode_legacy_signs", "load_exl3", "load_fixture",
           "rank_partition"]
__version__ = "0.3.0"
