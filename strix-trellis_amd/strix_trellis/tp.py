"""Two-rank tensor-parallel views of EXL3 groups, made at load time.

The entry point is the reference's ``rank_partition(tensor, site, rank,
bias_rank=0)`` (docs/LOADER.md, "Views by TP rank"); the site table holds the
shapes and rates of the mix-B / expert-TP layout it partitions.  Per site a
rank gets

* ``output``: an H128-aligned half of the output columns; the ranks' outputs
  are concatenated in rank order;
* ``input``: an H128-aligned half of the input channels; the ranks' outputs
  are summed, so only ``bias_rank`` keeps the bias;
* ``replicate``: the whole group.

Weights stay compressed (views of the tiles).  Only a complete group of the
site's shape is accepted, so a rank view is never partitioned again.
"""
from typing import NamedTuple

import numpy as np

from .loader import Exl3Tensor


class Site(NamedTuple):
    inputs: int
    outputs: int
    axis: str           # "output", "input" or "replicate"
    rates: tuple        # whole-bit rates the site's groups use


# The partitioned model's sites (facts about the model, as the reference lists them).
SITES = {
    "q_b": Site(1280, 32768, "output", (4, 5)),
    "o_b": Site(8192, 5120, "input", (4, 5)),
    "shared_gate": Site(5120, 2304, "output", (4, 5)),
    "shared_up": Site(5120, 2304, "output", (4, 5)),
    "shared_down": Site(2304, 5120, "input", (4, 5)),
    "q_a": Site(5120, 1280, "replicate", (4, 5)),
    "kv": Site(5120, 512, "replicate", (4, 5)),
    "expert_gate": Site(5120, 2304, "output", (2, 3)),
    "expert_up": Site(5120, 2304, "output", (2, 3)),
    "expert_down": Site(2304, 5120, "input", (2, 3)),
}


def _is_vector(values, size, itemsize):
    return (isinstance(values, np.ndarray) and values.dtype.kind == "f" and values.dtype.itemsize == itemsize
            and values.shape == (size,) and bool(np.isfinite(values).all()))


def _require_complete(tensor, name, site):
    """The group is a whole, folded-scale mul1 group of the site's shape."""
    if not isinstance(tensor, Exl3Tensor):
        raise ValueError("rank_partition takes an Exl3Tensor")
    if tensor.codebook != "mul1" or tensor.bits not in site.rates:
        raise ValueError(f"Site {name} takes mul1 groups at bitrates {site.rates}")
    want = (site.inputs // 16, site.outputs // 16, 16 * int(tensor.bits))
    tr = tensor.trellis
    if not (isinstance(tr, np.ndarray) and tr.dtype.kind == "i" and tr.dtype.itemsize == 2 and tr.shape == want):
        raise ValueError(f"Site {name} takes a complete I16 trellis of I={site.inputs}, N={site.outputs}")
    checks = (("suh", tensor.suh, site.inputs, 2), ("svh", tensor.svh, site.outputs, 2))
    for label, values, size, itemsize in checks:
        if not _is_vector(values, size, itemsize):
            raise ValueError(f"Site {name}: invalid folded F16 {label}")
    if tensor.bias is not None and not _is_vector(tensor.bias, site.outputs, 4):
        raise ValueError(f"Site {name}: invalid F32 bias")


def rank_partition(tensor, site, rank, *, bias_rank=0):
    """Rank ``rank`` (0 or 1) of a complete EXL3 group of TP site ``site``."""
    if type(site) is not str or site not in SITES:
        raise ValueError("Unknown TP site")
    for label, value in (("rank", rank), ("bias_rank", bias_rank)):
        if type(value) is not int or value not in (0, 1):
            raise ValueError(f"{label} must be the integer 0 or 1")
    spec = SITES[site]
    _require_complete(tensor, site, spec)
    if spec.axis == "output":
        half = spec.outputs // 2
        return tensor.slice_outputs(rank * half, (rank + 1) * half)
    if spec.axis == "input":
        half = spec.inputs // 2
        return tensor.slice_inputs(rank * half, (rank + 1) * half, include_bias=rank == bias_rank)
    return tensor
