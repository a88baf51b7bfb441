"""CPU tests of the two-rank TP views (strix_trellis.tp.rank_partition).

Groups are full site shapes built from broadcast (zero-copy) trellis arrays.
Checks: the axis each site splits, H128 alignment, the bias going to exactly
one input rank, replication returning the group itself, the rate / codebook
/ shape validation, and that a rank view is not accepted again."""
import numpy as np
import pytest

from strix_trellis.loader import Exl3Tensor
from strix_trellis.tp import SITES, rank_partition


def group(site, bits=None, codebook="mul1", bias=True):
    I, N, _, rates = SITES[site]
    bits = bits or rates[0]
    tr = np.broadcast_to(np.arange(16 * bits, dtype=np.int16), (I // 16, N // 16, 16 * bits))
    suh = np.linspace(-1, 1, I).astype(np.float16)
    svh = np.linspace(0.5, 1.5, N).astype(np.float16)
    b = np.arange(N, dtype=np.float32) if bias else None
    return Exl3Tensor(tr, suh, svh, float(bits), codebook, b, "mem", site)


@pytest.mark.parametrize("site", sorted(SITES))
def test_sites_split_the_documented_axis(site):
    I, N, axis, _ = SITES[site]
    g = group(site)
    r0, r1 = rank_partition(g, site, 0), rank_partition(g, site, 1)
    if axis == "replicate":
        assert r0 is g and r1 is g
        return
    if axis == "output":
        assert (r0.input_size, r0.output_size) == (I, N // 2) == (r1.input_size, r1.output_size)
        np.testing.assert_array_equal(np.concatenate([r0.svh, r1.svh]), g.svh)
        np.testing.assert_array_equal(np.concatenate([r0.bias, r1.bias]), g.bias)
        np.testing.assert_array_equal(np.concatenate([r0.trellis, r1.trellis], axis=1), g.trellis)
    else:
        assert (r0.input_size, r0.output_size) == (I // 2, N) == (r1.input_size, r1.output_size)
        np.testing.assert_array_equal(np.concatenate([r0.suh, r1.suh]), g.suh)
        np.testing.assert_array_equal(np.concatenate([r0.trellis, r1.trellis], axis=0), g.trellis)
        assert r0.bias is g.bias and r1.bias is None
        b1 = rank_partition(g, site, 1, bias_rank=1)
        assert b1.bias is g.bias and rank_partition(g, site, 0, bias_rank=1).bias is None
    assert r0.input_size % 128 == 0 and r0.output_size % 128 == 0
    with pytest.raises(ValueError):
        rank_partition(r0, site, 0)          # a rank view is not a complete group


def test_validation():
    g = group("q_b")
    for bad in (("nope", 0), ("q_b", 2), ("q_b", True), ("q_b", 1.0)):
        with pytest.raises(ValueError):
            rank_partition(g, *bad)
    with pytest.raises(ValueError):
        rank_partition(g, "q_b", 0, bias_rank=2)
    with pytest.raises(ValueError, match="mul1"):
        rank_partition(group("expert_up", bits=4), "expert_up", 0)
    with pytest.raises(ValueError, match="mul1"):
        rank_partition(group("o_b", codebook="mcg"), "o_b", 0)
    with pytest.raises(ValueError, match="complete"):
        rank_partition(group("kv"), "q_a", 0)
    bad_scale = group("kv")
    bad_scale.svh.flags.writeable = True
    bad_scale.svh[3] = np.inf
    with pytest.raises(ValueError, match="svh"):
        rank_partition(bad_scale, "kv", 0)
    with pytest.raises(ValueError):
        rank_partition("not a group", "kv", 0)
