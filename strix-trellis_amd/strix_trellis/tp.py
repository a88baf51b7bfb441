"""Two-rank tensor-parallel views of EXL3 groups, made at load time.

Same entry point as the reference (python/strix_trellis/tp.py:55-83,
``rank_partition``; docs/LOADER.md "Views by TP rank"): for the sites of the
mix-B / expert-TP layout (the site table below, reference tp.py:13-25) rank 0
or 1 gets

* an H128-aligned half of the output columns (``q_b``, ``*_gate``, ``*_up``);
  the ranks' outputs are concatenated in rank order;
* an H128-aligned half of the input channels (``o_b``, ``*_down``); the ranks'
  outputs are summed, and only ``bias_rank`` keeps the bias;
* or the whole group (``q_a``, ``kv``, replicated; never summed).

Weights stay compressed: the views slice the tiles (an output half repacks its
trellis only when exported).  The input group must be a complete group of the
site's shape -- a rank view is refused, so nothing is partitioned twice.
"""
import numpy as np

from .loader import Exl3Tensor

# site -> (input I, output N, partitioned axis, allowed whole-bit rates)
SITES = {
    "q_b": (1280, 32768, "output", (4, 5)),
    "o_b": (8192, 5120, "input", (4, 5)),
    "shared_gate": (5120, 2304, "output", (4, 5)),
    "shared_up": (5120, 2304, "output", (4, 5)),
    "shared_down": (2304, 5120, "input", (4, 5)),
    "q_a": (5120, 1280, "replicate", (4, 5)),
    "kv": (5120, 512, "replicate", (4, 5)),
    "expert_gate": (5120, 2304, "output", (2, 3)),
    "expert_up": (5120, 2304, "output", (2, 3)),
    "expert_down": (2304, 5120, "input", (2, 3)),
}


def _float_vector(value, size, itemsize):
    return (isinstance(value, np.ndarray) and value.shape == (size,) and value.dtype.kind == "f"
            and value.dtype.itemsize == itemsize and bool(np.isfinite(value).all()))


def _check(tensor, site):
    if not isinstance(tensor, Exl3Tensor):
        raise ValueError("rank_partition requires an Exl3Tensor")
    I, N, axis, rates = SITES[site]
    if tensor.codebook != "mul1" or tensor.bits not in rates:
        raise ValueError(f"{site} requires mul1 at bitrates {rates}")
    tr = tensor.trellis
    if not isinstance(tr, np.ndarray) or tr.dtype.kind != "i" or tr.dtype.itemsize != 2 or \
            tr.shape != (I // 16, N // 16, int(tensor.bits) * 16):
        raise ValueError(f"{site} requires a complete I16 trellis for I={I}, N={N}")
    if not _float_vector(tensor.suh, I, 2):
        raise ValueError(f"Invalid folded F16 suh for {site}")
    if not _float_vector(tensor.svh, N, 2):
        raise ValueError(f"Invalid folded F16 svh for {site}")
    if tensor.bias is not None and not _float_vector(tensor.bias, N, 4):
        raise ValueError(f"Invalid F32 bias for {site}")
    return I, N, axis


def rank_partition(tensor, site, rank, *, bias_rank=0):
    """Rank `rank` (0 or 1) of a complete EXL3 group of TP site `site`."""
    if type(site) is not str or site not in SITES:
        raise ValueError("Unknown TP site")
    if type(rank) is not int or rank not in (0, 1):
        raise ValueError("rank must be the integer 0 or 1")
    if type(bias_rank) is not int or bias_rank not in (0, 1):
        raise ValueError("bias_rank must be the integer 0 or 1")
    I, N, axis = _check(tensor, site)
    if axis == "replicate":
        return tensor
    if axis == "output":
        half = N // 2
        return tensor.slice_outputs(rank * half, (rank + 1) * half)
    half = I // 2
    return tensor.slice_inputs(rank * half, (rank + 1) * half, include_bias=rank == bias_rank)
