"""Seeded synthetic EXL3 layers (the measurement inputs of the benchmark).

NumPy ``Generator(PCG64(seed))``, drawn in a fixed order: trellis, suh, svh,
(bias), then activations.  Every bit pattern of the trellis is a valid stream
(reference docs/FORMAT.md:58-59); svh folds a per-column scale ~U(0.5, 1.5)
into random signs, as EXL3 requires.
"""
import numpy as np

BASE_SEED = 20261201


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def layer(I, N, K, seed, bias=False):
    g = rng(seed)
    trellis = g.integers(0, 65536, (I // 16, N // 16, 16 * K), dtype=np.uint16)
    suh = g.choice(np.array([-1.0, 1.0]), I).astype(np.float16)
    svh = (g.choice(np.array([-1.0, 1.0]), N) * g.uniform(0.5, 1.5, N)).astype(np.float16)
    b = g.standard_normal(N).astype(np.float32) if bias else None
    return trellis, suh, svh, b


def activations(R, I, seed):
    """x = RN16(N(0,1)) carried as F32 (exact)."""
    return rng(seed).standard_normal((R, I)).astype(np.float16).astype(np.float32)


def gate_values(actual, reference):
    """(maxabs, nrmse) of an output against its reference; inf when not all finite."""
    a = np.asarray(actual, dtype=np.float64)
    r = np.asarray(reference, dtype=np.float64)
    if not np.isfinite(a).all():
        return float("inf"), float("inf")
    maxabs = float(np.max(np.abs(a - r))) if a.size else 0.0
    nrmse = float(np.sqrt(np.sum((a - r) ** 2) / max(np.sum(r ** 2), 1e-30)))
    return maxabs, nrmse


def gate(actual, reference):
    """Acceptance of a full operator output (reference docs/GPU_TESTS.md:124-143):
    maxabs <= 5e-4 * max(1, max|ref|) and nrmse <= 3e-5, all finite."""
    a = np.asarray(actual, dtype=np.float64)
    r = np.asarray(reference, dtype=np.float64)
    assert np.isfinite(a).all(), "nonfinite output"
    maxabs, nrmse = gate_values(a, r)
    limit = 5e-4 * max(1.0, float(np.max(np.abs(r))) if r.size else 1.0)
    assert maxabs <= limit, f"maxabs {maxabs:.3e} > {limit:.3e}"
    assert nrmse <= 3e-5, f"nrmse {nrmse:.3e} > 3e-5"
    return maxabs, nrmse


def moe_bank(E, I, H, K, seed, bias=False, bits=None):
    """E experts, each dict(gate=(trellis, suh, svh, bias, K), up=..., down=...):
    gate/up [I -> H], down [H -> I].  ``bits`` = (Kgate, Kup, Kdown) overrides K."""
    kg, ku, kd = bits or (K, K, K)
    bank = []
    for e in range(E):
        s = seed + 3 * e
        g = layer(I, H, kg, s, bias)
        u = layer(I, H, ku, s + 1, bias)
        d = layer(H, I, kd, s + 2, bias)
        bank.append({"gate": (*g, kg), "up": (*u, ku), "down": (*d, kd)})
    return bank


def routes(R, E, k, seed):
    """Per token k distinct experts drawn uniformly (choice without replacement),
    scores = float32 softmax of N(0,1) logits over the k selected."""
    g = rng(seed)
    ids = np.stack([g.choice(E, k, replace=False) for _ in range(R)]).astype(np.uint32)
    logits = g.standard_normal((R, k))
    sc = np.exp(logits - logits.max(axis=1, keepdims=True))
    sc = (sc / sc.sum(axis=1, keepdims=True)).astype(np.float32)
    return ids, sc
