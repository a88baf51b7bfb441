"""The routed-expert oracle: its exp and SwiGLU against FP64, and the block
against its FP64 algebraic form and its structural identities."""
import math

import numpy as np
import pytest

import synth
from oracle import linear, moe


def _ulp_err(got, exact):
    got = np.asarray(got, np.float64)
    exact = np.asarray(exact, np.float64)
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    return np.abs(got - exact) / ulp


def test_exp_constants_are_the_documented_splits():
    assert float(moe.LN2_HEAD) == 0.693145751953125
    # the head has at most 16 significant bits, so n * head is exact for |n| <= 256
    m, _ = math.frexp(float(moe.LN2_HEAD))
    assert (m * 2 ** 16).is_integer()
    assert abs(float(moe.LN2_HEAD) + float(moe.LN2_TAIL) - math.log(2)) < 1e-13
    assert moe.LOG2E.view(np.uint32) == 0x3FB8AA3B


def test_exp_within_two_ulp_of_fp64():
    x = np.concatenate([np.linspace(-87.0, 0.0, 400001, dtype=np.float64),
                        -np.logspace(-30, 1.9, 20001)]).astype(np.float32)
    got = moe.exp_nonpos(x)
    exact = np.exp(x.astype(np.float64))
    assert float(np.max(_ulp_err(got, exact))) <= 2.0
    # subnormal results: absolute error within one subnormal step (2**-149) or two ulp
    xs = np.linspace(-103.9, -87.5, 20001, dtype=np.float32)
    err = np.abs(moe.exp_nonpos(xs).astype(np.float64) - np.exp(xs.astype(np.float64)))
    assert float(np.max(err)) <= 2.0 * 2.0 ** -149 + 2e-7 * float(np.max(np.exp(xs.astype(np.float64))))


def test_exp_special_values():
    x = np.array([0.0, -0.0, -np.inf, np.nan, -104.5, -1e-45], np.float32)
    got = moe.exp_nonpos(x)
    assert got[0] == 1.0 and got[1] == 1.0 and got[2] == 0.0 and np.isnan(got[3]) and got[4] == 0.0
    assert got[5] == 1.0


def test_swiglu_against_fp64():
    g = synth.rng(3).standard_normal(200000).astype(np.float32) * np.float32(6)
    u = synth.rng(4).standard_normal(200000).astype(np.float32)
    got = moe.swiglu(g, u).astype(np.float64)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    exact = g64 / (1.0 + np.exp(-g64)) * u64
    # exp <= 2 ulp, one division, two products: a few ulp of the result
    assert float(np.max(_ulp_err(got, exact))) <= 6.0
    # sign symmetry of the stable form: sigmoid(-g) = 1 - sigmoid(g) is not
    # assumed; SwiGLU(0, u) is exactly +0 or -0
    assert np.all(moe.swiglu(np.zeros(4, np.float32), np.ones(4, np.float32)) == 0)


def _tiny(K=2, E=5, I=256, H=128, R=3, k=2, seed=500, bias=True):
    bank = synth.moe_bank(E, I, H, K, seed, bias=bias)
    ids, sc = synth.routes(R, E, k, seed + 1)
    x = synth.activations(R, I, seed + 2)
    return bank, ids, sc, x


def test_block_matches_fp64_algebraic_form():
    bank, ids, sc, x = _tiny()
    cache = {}
    y, hidden = moe.moe_block(x, bank, ids, sc, cache=cache)
    # FP64 algebraic reference: every projection through linear.matmul (FP64)
    ref = np.zeros_like(y, dtype=np.float64)
    for r in range(ids.shape[0]):
        for s in range(ids.shape[1]):
            e = bank[int(ids[r, s])]
            lin = lambda v, w: linear.matmul(v, w[0], w[1], w[2], w[4], "mul1", w[3])
            g = lin(x[r:r + 1].astype(np.float64), e["gate"])[0]
            u = lin(x[r:r + 1].astype(np.float64), e["up"])[0]
            h = g / (1.0 + np.exp(-g)) * u
            ref[r] += float(sc[r, s]) * lin(h[None, :], e["down"])[0]
    err = np.max(np.abs(y - ref)) / np.max(np.abs(ref))
    assert err < 2e-3, err


def test_block_identities():
    bank, ids, sc, x = _tiny(R=4, k=3, E=6)
    cache = {}
    y, _ = moe.moe_block(x, bank, ids, sc, cache=cache)
    # tokens are independent
    y1, _ = moe.moe_block(x[2:3], bank, ids[2:3], sc[2:3], cache=cache)
    assert np.array_equal(y1.view(np.uint32), y[2:3].view(np.uint32))
    # a zero score contributes nothing: same bits as that slot's term absent
    sc0 = sc.copy()
    sc0[1, 2] = 0
    y0, _ = moe.moe_block(x, bank, ids, sc0, cache=cache)
    assert np.array_equal(y0[0].view(np.uint32), y[0].view(np.uint32))
    assert not np.array_equal(y0[1], y[1])
    # invalid tokens: repeated id, id outside the bank, negative or NaN score -> NaN row only
    for bad in ("dup", "range", "neg", "nan"):
        ib, sb = ids.copy(), sc.copy()
        if bad == "dup":
            ib[3, 1] = ib[3, 0]
        elif bad == "range":
            ib[3, 1] = len(bank)
        elif bad == "neg":
            sb[3, 1] = -0.5
        else:
            sb[3, 1] = np.nan
        yb, _ = moe.moe_block(x, bank, ib, sb, cache=cache)
        assert np.isnan(yb[3]).all()
        assert np.array_equal(yb[:3].view(np.uint32), y[:3].view(np.uint32))
    # alpha / beta on top of the same sum
    old = synth.rng(9).standard_normal(y.shape).astype(np.float32)
    yab, _ = moe.moe_block(x, bank, ids, sc, alpha=0.5, beta=-2.0, old=old, cache=cache)
    ref = (np.float32(0.5) * y).astype(np.float32)
    ref = (ref + (np.float32(-2.0) * old).astype(np.float32)).astype(np.float32)
    assert np.array_equal(yab.view(np.uint32), ref.view(np.uint32))


def test_down_finish_from_split_partials():
    """down_finish over S > 1 partials: exact splits of each core give the S = 1
    bits; the split sum starts at +0 in ascending order; entries of skipped
    routes are never read; a brute-force restatement over scalars agrees."""
    bank, ids, sc, x = _tiny(R=3, k=3, E=5)
    sc = sc.copy()
    sc[1, 2] = 0.0                          # a skipped slot
    ids = ids.copy()
    ids[2, 1] = ids[2, 0]                   # token 2 invalid (repeated id)
    _, hidden = moe.moe_block(x, bank, ids, sc, cache={})
    cores = moe.down_cores(hidden, bank, ids, sc)
    y1 = moe.down_combine(hidden, bank, ids, sc)
    assert np.array_equal(moe.down_finish(cores[:, :, None, :], bank, ids, sc).view(np.uint32), y1.view(np.uint32))
    assert np.isnan(y1[2]).all() and np.isfinite(y1[:2]).all()
    # Exact three-way splits: each core c as its top 8, next 8 and last 8
    # significant bits (same sign), so every partial sum is exact and the fold
    # reproduces c.
    g = synth.rng(77)
    S = 3
    P = np.zeros(cores.shape[:2] + (S, cores.shape[2]), np.float32)
    live = np.isfinite(cores)
    c64 = np.where(live, cores, 0).astype(np.float64)
    e = np.floor(np.log2(np.maximum(np.abs(c64), 1e-30)))
    hi = np.trunc(np.ldexp(c64, (7 - e).astype(np.int64)))
    hi = np.ldexp(hi, (e - 7).astype(np.int64))
    mid = np.ldexp(np.trunc(np.ldexp(c64 - hi, (15 - e).astype(np.int64))), (e - 15).astype(np.int64))
    P[:, :, 0] = hi.astype(np.float32)
    P[:, :, 1] = mid.astype(np.float32)
    P[:, :, 2] = (c64 - hi - mid).astype(np.float32)
    assert np.array_equal(P.astype(np.float64).sum(axis=2), c64)
    fold = ((P[:, :, 0] + P[:, :, 1]).astype(np.float32) + P[:, :, 2]).astype(np.float32)
    assert np.array_equal(fold[live].view(np.uint32), cores[live].view(np.uint32))
    # entries of the skipped slot and the invalid token are NaN: never read
    routed = live[:, :, 0]
    assert routed.sum() == routed.size - 1 - ids.shape[1]
    P[~routed] = np.nan
    yS = moe.down_finish(P, bank, ids, sc)
    same = (yS.view(np.uint32) == y1.view(np.uint32)) | (np.isnan(yS) & np.isnan(y1))
    assert same.all()
    # the split order is ascending from +0: a restatement over scalars for one
    # output of one token, against an order where the rounding differs
    Q = g.standard_normal(P.shape).astype(np.float32) * np.float32(1e3)
    Q[1, 0, 0] = np.float32(1e8)
    Q[1, 0, 1] = np.float32(-1e8)
    Q[1, 0, 2] = np.float32(0.75)
    Q[~routed] = np.nan
    yq = moe.down_finish(Q, bank, ids, sc)
    r = 1
    comb = np.zeros(yq.shape[1], np.float32)
    for s in range(3):
        if sc[r, s] == 0:
            continue
        core = np.zeros(Q.shape[3], np.float32)
        for u in range(S):
            core = (core + Q[r, s, u]).astype(np.float32)
        _, _, svh, bias, _ = bank[int(ids[r, s])]["down"]
        d = linear.output_stages_fp32(core[None, :], svh, bias)["output_fp32"][0]
        comb = (comb + (np.float32(sc[r, s]) * d).astype(np.float32)).astype(np.float32)
    assert np.array_equal(yq[r].view(np.uint32), comb.view(np.uint32))
    rev = Q.copy()
    rev[:, :, [0, 1, 2]] = Q[:, :, [2, 1, 0]]
    assert not np.array_equal(moe.down_finish(rev, bank, ids, sc)[r], yq[r])


def _order_pin_bank(k=4, I=128, H=128):
    """k experts whose down output stage is exactly H32 (svh = 1.0, no bias)."""
    bank = synth.moe_bank(k, I, H, 2, 600)
    for e in bank:
        tr, suh, svh, bias, K = e["down"]
        e["down"] = (tr, suh, np.ones_like(svh), None, K)
    return bank


def test_slot_combine_order_fixed_by_arithmetic():
    # The slot combine is RN32(score * d_s) added in ascending slot order from
    # +0.  Cores that are impulses (value v at element 0 of the 128-block)
    # make every element of d_s exactly v * c, c = RN32(1/sqrt(128)): the
    # butterflies only add zeros, and v is a power of two.  With unit scores
    # the terms are c*2^30, c, -c*2^30, 4c.  In ascending order c is absorbed
    # by c*2^30 (it needs 31 significant bits), the next term cancels, and the
    # sum is 4c exactly; descending order or a pairwise tree adds the 4c or
    # the c to -c*2^30 first, where it is absorbed, and ends at 0.
    c = np.float32(float.fromhex("0x1.6a09e6p-4"))
    k, I = 4, 128
    bank = _order_pin_bank(k, I)
    ids = np.arange(k, dtype=np.uint32)[None, :]
    sc = np.ones((1, k), np.float32)
    v = [2.0 ** 30, 1.0, -(2.0 ** 30), 4.0]
    P = np.zeros((1, k, 1, I), np.float32)
    for s in range(k):
        P[0, s, 0, 0] = v[s]
    y = moe.down_finish(P, bank, ids, sc)
    assert np.array_equal(y[0], np.full(I, np.float32(4) * c)), y[0][:4]
    # the other orders, evaluated in FP32 by hand, land on 0: the check above
    # tells ascending order apart from them
    t = [np.float32(x) * c for x in v]
    desc = np.float32(0)
    for x in reversed(t):
        desc = np.float32(desc + x)
    tree = np.float32(np.float32(t[0] + t[1]) + np.float32(t[2] + t[3]))
    assert desc == 0 and tree == 0
    # a zero score removes its slot: without slot 1 the sum is c*2^30 - c*2^30 + 4c
    sc0 = sc.copy()
    sc0[0, 1] = 0
    assert np.array_equal(moe.down_finish(P, bank, ids, sc0)[0], np.full(I, np.float32(4) * c))
    # scores scale terms exactly (powers of two): score 0.5 on slot 3 gives 2c
    sc3 = sc.copy()
    sc3[0, 3] = 0.5
    assert np.array_equal(moe.down_finish(P, bank, ids, sc3)[0], np.full(I, np.float32(2) * c))
