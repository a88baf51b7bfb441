"""Routed-expert (SwiGLU + ordered weighted top-k) block on top of ``linear``.

TEST INFRASTRUCTURE ONLY (see the package docstring).

Operator (reference docs/TP_RANK.md:64-76, include/strix_trellis.h:207-233):

    hidden[r, s] = SwiGLU(gate_e(x[r]), up_e(x[r]))          e = ids[r, s]
    y[r]         = alpha * sum_s score[r, s] * down_e(hidden[r, s]) + beta * y[r]

* every projection is the staged FP32 linear of ``linear.matmul_fp32_stages``
  (input stage, core, output stage with svh and bias), alpha 1, beta 0;
* SwiGLU = g * sigmoid(g) * u with the stable sigmoid (1/(1+e^-g) for g >= 0,
  e^g/(1+e^g) for g < 0; reference src/tp_moe_activation.hpp:46-60), each
  product rounded to FP32; ``exp`` is this library's own (below), because the
  reference's default uses the device ``expf``, whose bits are not specified;
* the slot sum starts at +0 and visits s = 0..k-1, adding RN32(score * value)
  with one FP32 rounding; an exactly zero score skips its term (reference
  src/tp_moe.hip:100-160);
* y = RN32(alpha * sum), then + RN32(beta * y_old) iff beta != 0;
* a token with an id outside the bank, a repeated id, or a non-finite or
  negative score gets an all-NaN row (reference src/tp_moe_routes.hpp:25-62).
"""
import math

import numpy as np

from . import codec, linear

F32 = np.float32

# exp(x), x <= 0: Cody-Waite reduction x = n*ln2 + r (ln2 = head + tail, head
# with 16 significant bits), degree-7 Taylor polynomial of exp(r) in Horner
# form, then two power-of-two factors.  Same single-precision operations, in
# the same order, as the device code, so the bits agree.
LOG2E = F32(1.44269504088896341)
LN2_HEAD = F32(0.693145751953125)
LN2_TAIL = F32(1.42860682030941723e-6)
INV_FACT = [F32(1) / F32(math.factorial(k)) for k in range(8)]


def _pow2(k):
    return ((k.astype(np.int64) + 127) << 23).astype(np.uint32).view(F32)


def exp_nonpos(x):
    """exp of float32 values <= 0 (NaN passes through), elementwise."""
    x = np.asarray(x, dtype=F32)
    with np.errstate(invalid="ignore", over="ignore", under="ignore"):
        safe = np.where((x == x) & (x >= F32(-104)), x, F32(0))
        n = np.rint(safe * LOG2E)
        r = (safe - n * LN2_HEAD) - n * LN2_TAIL
        p = np.full_like(r, INV_FACT[7])
        for k in range(6, -1, -1):
            p = p * r + INV_FACT[k]
        ni = n.astype(np.int64)
        n1 = np.trunc(ni / 2).astype(np.int64)     # C integer division truncates toward zero
        n2 = ni - n1
        out = (p * _pow2(n1)) * _pow2(n2)
    out = np.where(x < F32(-104), F32(0), out)
    return np.where(x == x, out, x).astype(F32)


def swiglu(g, u):
    """Activation of the gate/up finish, float32 elementwise."""
    g = np.asarray(g, dtype=F32)
    u = np.asarray(u, dtype=F32)
    neg = g < F32(0)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        ex = exp_nonpos(np.where(neg, g, -g))
        den = F32(1) + ex
        sig = np.where(neg, ex / den, F32(1) / den)
        act = g * sig
        return (act * u).astype(F32)


def token_valid(ids, scores, bank_count):
    """Per-token validity of [rows, k] routes (ids in range and distinct, scores finite >= 0)."""
    ids = np.asarray(ids)
    scores = np.asarray(scores, dtype=F32)
    ok = np.ones(ids.shape[0], dtype=bool)
    for r in range(ids.shape[0]):
        row = ids[r]
        if np.any(row >= bank_count) or len(set(row.tolist())) != row.size:
            ok[r] = False
        if not np.all(np.isfinite(scores[r])) or np.any(scores[r] < 0):
            ok[r] = False
    return ok


def projection(x_rows, w, cache=None, key=None):
    """Staged FP32 linear of ``w = (trellis, suh, svh, bias, K)``: [rows, I] -> [rows, N]."""
    trellis, suh, svh, bias, k = w
    q = None
    if cache is not None:
        q = cache.get(key)
        if q is None:
            q = cache[key] = codec.dequantize_rotated(trellis, k)
    return linear.matmul_fp32_stages(np.asarray(x_rows, F32), trellis, suh, svh, k, "mul1", bias,
                                     rotated=q)["output_fp32"]


def down_finish(partials, experts, ids, scores, alpha=1.0, beta=0.0, old=None):
    """The down finish from per-split core partials ``partials`` [rows, k, S, I]:
    per valid token, each non-zero-score slot's core is its S partials summed
    from +0 in ascending split order (FP32), then that expert's down output
    stage; the slot sum, alpha/beta and the NaN rows of invalid tokens as in
    ``down_combine``.  Entries of zero-score slots and invalid tokens are not
    read.  With S = 1 and the cores of ``linear.core_dot_fp32`` it is
    ``down_combine`` itself (which calls it so)."""
    P = np.asarray(partials, F32)
    ids = np.asarray(ids)
    scores = np.asarray(scores, F32)
    rows, k, S, I = P.shape
    valid = token_valid(ids, scores, len(experts))
    y = np.empty((rows, I), F32)
    for r in range(rows):
        if not valid[r]:
            y[r] = np.float32(np.nan)
            continue
        comb = np.zeros(I, F32)
        for s in range(k):
            sc = F32(scores[r, s])
            if sc == 0:
                continue
            core = np.zeros(I, F32)
            for u in range(S):
                core = (core + P[r, s, u]).astype(F32)
            _, _, svh, bias, _ = experts[int(ids[r, s])]["down"]
            d = linear.output_stages_fp32(core[None, :], svh, bias)["output_fp32"][0]
            comb = (comb + (sc * d).astype(F32)).astype(F32)
        out = (F32(alpha) * comb).astype(F32)
        if beta != 0:
            out = (out + (F32(beta) * np.asarray(old[r], F32)).astype(F32)).astype(F32)
        y[r] = out
    return y


def down_cores(hidden, experts, ids, scores, cache=None):
    """FP32 down cores [rows, k, I] of the computed routes (valid token,
    non-zero score) from hidden [rows, k, H]; NaN elsewhere."""
    hidden = np.asarray(hidden, F32)
    ids = np.asarray(ids)
    scores = np.asarray(scores, F32)
    rows, k = ids.shape
    I = experts[0]["down"][2].shape[0]       # down svh: [I]
    valid = token_valid(ids, scores, len(experts))
    cores = np.full((rows, k, I), np.nan, F32)
    for r in range(rows):
        for s in range(k):
            if not valid[r] or scores[r, s] == 0:
                continue
            e = int(ids[r, s])
            trellis, suh, svh, bias, kk = experts[e]["down"]
            q = None
            if cache is not None:
                q = cache.get((e, "down"))
                if q is None:
                    q = cache[(e, "down")] = codec.dequantize_rotated(trellis, kk)
            st = linear.matmul_fp32_stages(hidden[r, s][None, :], trellis, suh, svh, kk, "mul1", bias, rotated=q)
            cores[r, s] = st["core_fp32"][0]
    return cores


def down_combine(hidden, experts, ids, scores, alpha=1.0, beta=0.0, old=None, cache=None):
    """The down half alone: y from given hidden [rows, k, H] (invalid tokens -> NaN rows)."""
    cores = down_cores(hidden, experts, ids, scores, cache)
    return down_finish(cores[:, :, None, :], experts, ids, scores, alpha, beta, old)


def moe_block(x, experts, ids, scores, alpha=1.0, beta=0.0, old=None, cache=None):
    """Returns (y, hidden).  ``experts[i] = dict(gate=w, up=w, down=w)``; ids index ``experts``.

    hidden is [rows, k, H] with NaN where a route was not computed (invalid
    token or zero score).
    """
    x = np.asarray(x, F32)
    ids = np.asarray(ids)
    scores = np.asarray(scores, F32)
    rows, k = ids.shape
    H = experts[0]["gate"][2].shape[0]            # gate svh: [H]
    valid = token_valid(ids, scores, len(experts))
    hidden = np.full((rows, k, H), np.nan, F32)
    for r in range(rows):
        for s in range(k):
            if not valid[r] or scores[r, s] == 0:
                continue
            e = int(ids[r, s])
            g = projection(x[r:r + 1], experts[e]["gate"], cache, (e, "gate"))[0]
            u = projection(x[r:r + 1], experts[e]["up"], cache, (e, "up"))[0]
            hidden[r, s] = swiglu(g, u)
    return down_combine(hidden, experts, ids, scores, alpha, beta, old, cache), hidden
