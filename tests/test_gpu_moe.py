"""GPU parity of the routed-expert block (strix_tp_moe_* plans) through the C ABI.

Bars:
* the activation is bit-exact to the oracle's SwiGLU (its own exp);
* hidden and the block output meet the reference GPU gate against the staged
  FP32 oracle (the projections' cores accumulate in the GPU order);
* identities that fix the bits exactly: host-route plan == device-route plan,
  a token's output does not depend on the other tokens or on the order of the
  expert array, a zero score removes its slot, invalid tokens give NaN rows
  and leave the others untouched, alpha/beta apply on top of the same sum,
  replays of a captured graph follow routes rewritten in place.
"""
import numpy as np
import pytest

import synth
from oracle import moe

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from strix_trellis import abi, runtime  # noqa: E402

DEV = "cuda:0"


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    c = runtime.Context(0)
    yield c
    torch.cuda.synchronize()


def _weights(ctx, bank):
    out = []
    for e in bank:
        ws = []
        for p in ("gate", "up", "down"):
            tr, suh, svh, b, _ = e[p]
            ws.append(runtime.Weights(ctx, tr, suh, svh, b, "mul1"))
        out.append(tuple(ws))
    return out


def _destroy(ws):
    for t in ws:
        for w in t:
            w.destroy()


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _run(ctx, ws, x, ids, sc, alpha=1.0, beta=0.0, old=None, device=False, expert_ids=None):
    y = _dev(old) if old is not None else torch.full((x.shape[0], x.shape[1]), float("nan"), device=DEV)
    xd = _dev(x)
    if device:
        di = _dev(ids.astype(np.int32))
        ds = _dev(sc.astype(np.float32))
        plan = runtime.MoePlan(ctx, ws, xd, y, device_ids=di, device_scores=ds, alpha=alpha, beta=beta)
    else:
        plan = runtime.MoePlan(ctx, ws, xd, y, ids=ids, scores=sc, expert_ids=expert_ids, alpha=alpha, beta=beta)
    plan.submit()
    torch.cuda.synchronize()
    out, hidden = y.cpu().numpy(), plan.hidden.cpu().numpy()
    plan.destroy()
    return out, hidden


def test_swiglu_bit_exact(ctx):
    g = synth.rng(21).standard_normal(1 << 18).astype(np.float32) * np.float32(8)
    u = synth.rng(22).standard_normal(1 << 18).astype(np.float32)
    special = np.array([0.0, -0.0, 1e-40, -1e-40, 88.0, -88.0, 103.0, -103.0, 104.5, -104.5, 200.0, -200.0,
                        np.inf, -np.inf, np.nan, 1.0, -1.0, 3.4e38, -3.4e38], np.float32)
    g[:special.size] = special
    u[:special.size] = 1.5
    h = runtime.swiglu(ctx, _dev(g), _dev(u)).cpu().numpy()
    ref = moe.swiglu(g, u)
    same = (h.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(h) & np.isnan(ref))
    assert same.all(), f"{np.count_nonzero(~same)} differ, first at {np.flatnonzero(~same)[:4]}"


MOE_CASES = [
    # (E, I, H, R, k, bits (gate, up, down), bias)
    (6, 256, 128, 3, 2, (2, 2, 2), True),
    (8, 512, 256, 4, 3, (3, 2, 3), False),
    (5, 256, 384, 2, 4, (2, 3, 2), True),
    (12, 1024, 256, 8, 6, (2, 2, 3), False),
]


@pytest.mark.parametrize("E,I,H,R,k,bits,bias", MOE_CASES)
def test_block_matches_oracle(ctx, E, I, H, R, k, bits, bias):
    print(f"moe E={E} I={I} H={H} R={R} k={k} bits={bits} bias={bias}", flush=True)
    seed = 9000 + E + R
    bank = synth.moe_bank(E, I, H, 2, seed, bias=bias, bits=bits)
    ids, sc = synth.routes(R, E, k, seed + 50)
    used = sorted(set(ids.ravel().tolist()))
    # host plans take the exact union: relabel to the used experts
    sub = [bank[e] for e in used]
    remap = {e: i for i, e in enumerate(used)}
    ids_u = np.vectorize(remap.get)(ids).astype(np.uint32)
    x = synth.activations(R, I, seed + 60)
    ws = _weights(ctx, sub)
    y, hidden = _run(ctx, ws, x, ids_u, sc)
    cache = {}
    ref, href = moe.moe_block(x, sub, ids_u, sc, cache=cache)
    # hidden = SwiGLU of two projections: twice the single-linear nrmse bar
    a, r = hidden.reshape(-1, H).astype(np.float64), href.reshape(-1, H).astype(np.float64)
    assert np.isfinite(a).all()
    nrmse = np.sqrt(np.sum((a - r) ** 2) / np.sum(r ** 2))
    assert np.max(np.abs(a - r)) <= 5e-4 * max(1.0, np.max(np.abs(r))) and nrmse <= 6e-5, nrmse
    # the down half from the GPU's own hidden: the single-linear gate
    synth.gate(y, moe.down_combine(hidden, sub, ids_u, sc, cache=cache))
    # the whole chain (three projections) against the oracle: max-rel-err 1e-3
    assert np.max(np.abs(y - ref)) <= 1e-3 * np.max(np.abs(ref))
    # the same routes through a device bank of all E experts give the same bits
    wall = _weights(ctx, bank)
    yd, _ = _run(ctx, wall, x, ids, sc, device=True)
    assert np.array_equal(yd.view(np.uint32), y.view(np.uint32))
    _destroy(ws)
    _destroy(wall)


def test_block_identities(ctx):
    E, I, H, R, k = 10, 512, 256, 6, 3
    bank = synth.moe_bank(E, I, H, 2, 777, bias=True)
    ids, sc = synth.routes(R, E, k, 778)
    x = synth.activations(R, I, 779)
    ws = _weights(ctx, bank)
    y, _ = _run(ctx, ws, x, ids, sc, device=True)
    # token independence: each token alone gives its own bits
    for r in (0, 3, 5):
        yr, _ = _run(ctx, ws, x[r:r + 1], ids[r:r + 1], sc[r:r + 1], device=True)
        assert np.array_equal(yr.view(np.uint32), y[r:r + 1].view(np.uint32)), r
    # the host plan with the expert array permuted (ids name experts by expert_id)
    used = sorted(set(ids.ravel().tolist()))
    order = used[::-1]
    wsub = [ws[e] for e in order]
    yh, _ = _run(ctx, wsub, x, ids, sc, expert_ids=order)
    assert np.array_equal(yh.view(np.uint32), y.view(np.uint32))
    # zero score: the slot disappears, other tokens unchanged
    sc0 = sc.copy()
    sc0[2, 1] = 0.0
    y0, _ = _run(ctx, ws, x, ids, sc0, device=True)
    ref0, _ = moe.moe_block(x, bank, ids, sc0, cache={})
    assert np.max(np.abs(y0 - ref0)) <= 1e-3 * np.max(np.abs(ref0))
    keep = [r for r in range(R) if r != 2]
    assert np.array_equal(y0[keep].view(np.uint32), y[keep].view(np.uint32))
    # invalid device routes -> NaN rows only
    for bad in ("dup", "range", "neg", "nan"):
        ib, sb = ids.copy(), sc.copy()
        if bad == "dup":
            ib[4, 2] = ib[4, 0]
        elif bad == "range":
            ib[4, 2] = 1000
        elif bad == "neg":
            sb[4, 2] = -1.0
        else:
            sb[4, 2] = np.nan
        yb, _ = _run(ctx, ws, x, ib, sb, device=True)
        assert np.isnan(yb[4]).all(), bad
        others = [r for r in range(R) if r != 4]
        assert np.array_equal(yb[others].view(np.uint32), y[others].view(np.uint32)), bad
    # alpha / beta exactly on top of the same slot sum
    old = synth.rng(5).standard_normal((R, I)).astype(np.float32)
    yab, _ = _run(ctx, ws, x, ids, sc, alpha=0.75, beta=-1.5, old=old, device=True)
    ref = (np.float32(0.75) * y).astype(np.float32)
    ref = (ref + (np.float32(-1.5) * old).astype(np.float32)).astype(np.float32)
    assert np.array_equal(yab.view(np.uint32), ref.view(np.uint32))
    _destroy(ws)


def test_device_routes_rewritten_between_graph_replays(ctx):
    E, I, H, R, k = 8, 256, 128, 4, 2
    bank = synth.moe_bank(E, I, H, 2, 333)
    ws = _weights(ctx, bank)
    x = synth.activations(R, I, 334)
    xd = _dev(x)
    y = torch.empty((R, I), device=DEV)
    routes = [synth.routes(R, E, k, 340 + i) for i in range(3)]
    di = _dev(routes[0][0].astype(np.int32))
    ds = _dev(routes[0][1])
    stream = torch.cuda.Stream()
    plan = runtime.MoePlan(ctx, ws, xd, y, device_ids=di, device_scores=ds, stream=stream)
    expected = [_run(ctx, ws, x, i, s, device=True)[0] for i, s in routes]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        plan.submit()
    torch.cuda.synchronize()
    for rep in range(6):
        i, s = routes[rep % 3]
        di.copy_(_dev(i.astype(np.int32)))
        ds.copy_(_dev(s))
        torch.cuda.synchronize()
        y.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), expected[rep % 3].view(np.uint32)), rep
    del graph
    plan.destroy()
    _destroy(ws)


def test_staged_entry_points_and_validation(ctx):
    E, I, H, R, k = 6, 256, 128, 2, 3
    bank = synth.moe_bank(E, I, H, 2, 444)
    ws = _weights(ctx, bank)
    ids, sc = synth.routes(R, E, k, 445)
    x = synth.activations(R, I, 446)
    full, hidden = _run(ctx, ws, x, ids, sc, device=True)
    y = torch.empty((R, I), device=DEV)
    plan = runtime.MoePlan(ctx, ws, _dev(x), y, device_ids=_dev(ids.astype(np.int32)), device_scores=_dev(sc))
    plan.gate_up()
    plan.down()
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), full.view(np.uint32))
    plan.destroy()
    # a staged down call reads hidden as the caller left it: with hidden
    # zeroed between the stages every core and (bias-free) output is zero
    wsp = torch.empty(R * k * H, dtype=torch.float32, device=DEV)
    plan = runtime.MoePlan(ctx, ws, _dev(x), y, device_ids=_dev(ids.astype(np.int32)), device_scores=_dev(sc),
                           workspace=wsp)
    plan.gate_up()
    wsp.zero_()
    y.fill_(float("nan"))
    plan.down()
    torch.cuda.synchronize()
    assert not torch.any(y.view(torch.int32) != 0)
    # and the whole block again matches the two-stage result
    plan.submit()
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), full.view(np.uint32))
    # weights retained by a plan cannot be destroyed
    assert ctx.lib.strix_weights_destroy(ws[0][0].handle) != 0
    plan.destroy()
    # host routes must name exactly the given experts: 12 experts cannot all
    # be used by 2 x 3 routes
    wbig = _weights(ctx, synth.moe_bank(12, I, H, 2, 448))
    with pytest.raises(abi.StrixError):
        runtime.MoePlan(ctx, wbig, _dev(x), y, ids=ids, scores=sc)
    # k > 8 routes per token is rejected
    ids9, sc9 = synth.routes(1, 12, 9, 447)
    with pytest.raises(abi.StrixError):
        runtime.MoePlan(ctx, wbig, _dev(x[:1]), y[:1], device_ids=_dev(ids9.astype(np.int32)),
                        device_scores=_dev(sc9))
    _destroy(ws)
    _destroy(wbig)


def _same_bits(a, b):
    """Bitwise equality where NaN matches NaN."""
    return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


def test_split_plan_checkpoints(ctx):
    """Split plans keep the down core's per-split partials P [rows, k, S, I] in
    the workspace (S = 4 here, the reference's partition; the plain plan's
    own split count differs).  The fused down and the staged core write the same P; the
    route-alone core writes it again without the expert grouping; the staged
    finish reproduces the fused output from P and, on any P, the oracle's
    finish bit for bit; P's split sums meet the core's FP64 bound.  Plain plans
    refuse the staged down."""
    from oracle import codec, linear
    E, I, H, R, k = 6, 256, 2048, 3, 3
    print(f"moe split plan E={E} I={I} H={H} R={R} k={k}", flush=True)
    bank = synth.moe_bank(E, I, H, 2, 555, bias=True)
    ws = _weights(ctx, bank)
    ids, sc = synth.routes(R, E, k, 556)
    sc[0, 1] = 0.0            # a skipped slot
    ids[2, 2] = ids[2, 0]     # token 2 is invalid: NaN row
    x = synth.activations(R, I, 557)
    routed = np.ones((R, k), bool)
    routed[0, 1] = False
    routed[2] = False
    y_plain, _ = _run(ctx, ws, x, ids, sc, device=True)
    assert np.isnan(y_plain[2]).all() and np.isfinite(y_plain[:2]).all()

    y = torch.full((R, I), float("nan"), device=DEV)
    plan = runtime.MoePlan(ctx, ws, _dev(x), y, device_ids=_dev(ids.astype(np.int32)), device_scores=_dev(sc),
                           split=True)
    S = plan.partials.shape[2]
    assert plan.partials.shape == (R, k, S, I) and S == 4
    plan.submit()
    torch.cuda.synchronize()
    y_full, P_full = y.cpu().numpy(), plan.partials.cpu().numpy()
    hidden = plan.hidden.cpu().numpy()
    assert np.isfinite(P_full[routed]).all()
    # the fused split output is the oracle's finish of its own planes; the
    # plain plan folds the down core in another split count, so it agrees
    # within the reference GPU gate, NaN row included
    assert _same_bits(y_full, moe.down_finish(P_full, bank, ids, sc))
    assert np.isnan(y_full[2]).all()
    synth.gate(y_full[:2], y_plain[:2].astype(np.float64))

    # the staged core writes the same P for every computed route, nothing else
    plan.partials.fill_(float("nan"))
    plan.gate_up()
    plan.down_core()
    torch.cuda.synchronize()
    P_core = plan.partials.cpu().numpy()
    assert _same_bits(P_core[routed], P_full[routed])
    assert np.isnan(P_core[~routed]).all()
    # the staged finish from P gives the fused output, NaN row included
    y.fill_(0.0)
    plan.down_finish()
    torch.cuda.synchronize()
    assert _same_bits(y.cpu().numpy(), y_full)
    # route-alone core: the same P without the expert grouping
    plan.partials.fill_(float("nan"))
    plan.down_reference_core()
    torch.cuda.synchronize()
    P_ref = plan.partials.cpu().numpy()
    assert _same_bits(P_ref[routed], P_full[routed])
    assert np.isnan(P_ref[~routed]).all()

    # P against the oracle: each computed route's split sum (ascending from +0)
    # within the FP64 bound of its core, from the GPU's own hidden
    for r in range(R):
        for s in range(k):
            if not routed[r, s]:
                continue
            tr, suh, _, _, kk = bank[int(ids[r, s])]["down"]
            a = linear.input_stages_fp32(hidden[r, s][None, :], suh)["core_input_fp16"]
            q = codec.dequantize_rotated(tr, kk)
            fold = np.zeros(I, np.float32)
            for u in range(S):
                fold = (fold + P_full[r, s, u]).astype(np.float32)
            assert np.all(np.abs(fold - linear.core_exact_f64(a, q)[0]) <= linear.gamma_bound(a, q)[0]), (r, s)

    # the staged finish on an arbitrary P follows the oracle's finish bit for bit
    g = synth.rng(558)
    Q = (g.standard_normal((R, k, S, I)) * 50).astype(np.float32)
    plan.partials.copy_(_dev(Q))
    y.fill_(0.0)
    plan.down_finish()
    torch.cuda.synchronize()
    assert _same_bits(y.cpu().numpy(), moe.down_finish(Q, bank, ids, sc))
    plan.destroy()

    # a host-route split plan over the used experts gives the same P and output
    used = sorted(set(ids[:2].ravel().tolist()))
    remap = {e: i for i, e in enumerate(used)}
    rows_ok = [0, 1]
    ih = np.vectorize(remap.get)(ids[rows_ok]).astype(np.uint32)
    yh = torch.full((2, I), float("nan"), device=DEV)
    hp = runtime.MoePlan(ctx, [ws[e] for e in used], _dev(x[rows_ok]), yh, ids=ih, scores=sc[rows_ok], split=True)
    hp.submit()
    torch.cuda.synchronize()
    assert _same_bits(yh.cpu().numpy(), y_full[rows_ok])
    assert _same_bits(hp.partials.cpu().numpy()[routed[rows_ok]], P_full[rows_ok][routed[rows_ok]])
    hp.destroy()

    # plain plans have no P: the staged down is refused
    yp = torch.empty((R, I), device=DEV)
    pp = runtime.MoePlan(ctx, ws, _dev(x), yp, device_ids=_dev(ids.astype(np.int32)), device_scores=_dev(sc))
    assert pp.partials is None
    for fn in (pp.down_core, pp.down_finish, pp.down_reference_core):
        with pytest.raises(abi.StrixError):
            fn()
    pp.destroy()
    _destroy(ws)



def test_split_plan_reference_partition(ctx):
    """At the reference's split geometry (5120 <-> 1152, top-6) a split plan's
    P is [rows, 6, 4, 5120], split u over the down input's blocks
    [18 u, 18 u + 18) (reference src/tp_fused_layout.hpp:19-24): each plane
    meets the FP64 bound of the core over its own 288 channels alone, so a
    shifted or resized partition fails.  Split u = 1 and 3 start inside a
    128-channel group.  The staged finish of reference-layout planes follows
    the oracle's finish bit for bit, and the fused output equals the plain
    plan's up to the fold order (planes vs. one sum)."""
    from oracle import codec, linear
    E, I, H, R, k = 8, 5120, 1152, 2, 6
    print(f"moe split plan reference partition E={E} I={I} H={H} R={R} k={k}", flush=True)
    bank = synth.moe_bank(E, I, H, 2, 731, bias=True)
    ws = _weights(ctx, bank)
    ids, sc = synth.routes(R, E, k, 732)
    x = synth.activations(R, I, 733)
    y = torch.full((R, I), float("nan"), device=DEV)
    plan = runtime.MoePlan(ctx, ws, _dev(x), y, device_ids=_dev(ids.astype(np.int32)), device_scores=_dev(sc),
                           split=True)
    assert plan.partials.shape == (R, k, 4, I)
    plan.submit()
    torch.cuda.synchronize()
    y_full, P = y.cpu().numpy(), plan.partials.cpu().numpy()
    hidden = plan.hidden.cpu().numpy()
    assert np.isfinite(P).all() and np.isfinite(y_full).all()
    # the staged core writes the same planes
    plan.partials.fill_(float("nan"))
    plan.down_core()
    torch.cuda.synchronize()
    assert _same_bits(plan.partials.cpu().numpy(), P)

    qs = {}
    for r in range(R):
        for s in range(k):
            e = int(ids[r, s])
            tr, suh, _, _, kk = bank[e]["down"]
            if e not in qs:
                qs[e] = codec.dequantize_rotated(tr, kk)
            a = linear.input_stages_fp32(hidden[r, s][None, :], suh)["core_input_fp16"]
            for u in range(4):
                c0, c1 = 288 * u, 288 * (u + 1)
                exact = linear.core_exact_f64(a[:, c0:c1], qs[e][c0:c1])[0]
                bound = linear.gamma_bound(a[:, c0:c1], qs[e][c0:c1])[0]
                assert np.all(np.abs(P[r, s, u] - exact) <= bound), (r, s, u)
    # the finish from the planes as they are is the oracle's finish
    assert _same_bits(y_full, moe.down_finish(P, bank, ids, sc))
    g = synth.rng(734)
    Q = (g.standard_normal((R, k, 4, I)) * 50).astype(np.float32)
    plan.partials.copy_(_dev(Q))
    y.fill_(0.0)
    plan.down_finish()
    torch.cuda.synchronize()
    assert _same_bits(y.cpu().numpy(), moe.down_finish(Q, bank, ids, sc))
    plan.destroy()
    # against the plain plan (one down sum): the same hidden, outputs within
    # the reference GPU gate of each other
    y_plain, h_plain = _run(ctx, ws, x, ids, sc, device=True)
    assert _same_bits(h_plain, hidden)
    synth.gate(y_full, y_plain.astype(np.float64))
    _destroy(ws)

def test_down_finish_slot_order_fixed_by_arithmetic(ctx):
    """The device's slot combine is ascending from +0, pinned by arithmetic
    rather than by the oracle's restatement: with svh = 1, no bias and impulse
    cores (split 0 holds v at element 0, the other splits +0), every element of
    slot s's output is exactly v_s * c, c = RN32(1/sqrt(128)).  Terms c*2^30,
    c, -c*2^30, 4c at unit scores sum to exactly 4c in ascending order from +0
    (c is absorbed by c*2^30, which then cancels) and to 0 in descending order
    or as a pairwise tree.  Zero scores drop slots; power-of-two scores scale
    exactly."""
    k, I, H = 4, 128, 2048
    print(f"moe slot order pin k={k} I={I} H={H}", flush=True)
    bank = synth.moe_bank(k, I, H, 2, 600)
    for e in bank:
        tr, suh, svh, _, K = e["down"]
        e["down"] = (tr, suh, np.ones_like(svh), None, K)
    ws = _weights(ctx, bank)
    c = np.float32(float.fromhex("0x1.6a09e6p-4"))
    ids = np.arange(k, dtype=np.int32)[None, :]
    x = synth.activations(1, I, 601)
    for scores, expect in (([1.0, 1.0, 1.0, 1.0], 4 * c), ([1.0, 0.0, 1.0, 1.0], 4 * c),
                           ([1.0, 1.0, 1.0, 0.5], 2 * c)):
        sc = np.array([scores], np.float32)
        y = torch.full((1, I), float("nan"), device=DEV)
        plan = runtime.MoePlan(ctx, ws, _dev(x), y, device_ids=_dev(ids), device_scores=_dev(sc), split=True)
        S = plan.partials.shape[2]
        P = np.zeros((1, k, S, I), np.float32)
        for s, v in enumerate((2.0 ** 30, 1.0, -(2.0 ** 30), 4.0)):
            P[0, s, 0, 0] = v
        plan.partials.copy_(_dev(P))
        plan.down_finish()
        torch.cuda.synchronize()
        got = y.cpu().numpy()[0]
        plan.destroy()
        assert np.array_equal(got, np.full(I, np.float32(expect))), (scores, got[:4])
    for t in ws:
        for w in t:
            w.destroy()
