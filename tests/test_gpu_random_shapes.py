"""Bit-exact parity of MoeLayer::forward over seeded random layer shapes.

Each case draws a format, hidden and intermediate sizes (multiples of 32,
not of 64 or 2048), an expert count, a top-k, a token count (1 to 80, so
the decode pass, the grouped path and the router's many-token kernel all
occur) and whether router logits are given, and compares every token's
routes, weights and output with the oracle's token-at-a-time forward.  The
draws reach combinations the hand-picked tests do not: wave counts, two
tiles per work-group, chain rings, partial tiles and chunks.
"""
import numpy as np
import pytest

import hale_moe as H
import oracle as O

pytestmark = pytest.mark.gpu

REL_L2 = 1e-5


def same_bits(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and bool((a.view(np.uint32) == b.view(np.uint32)).all())


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def draw(seed):
    """One layer shape and call; E * H * I kept under 2^26 weights so the
    oracle builds the layer in seconds."""
    rng = np.random.default_rng(seed)
    while True:
        dtype = [O.Q8_0, O.Q4_0][rng.integers(2)]
        hid = 32 * int(rng.integers(1, 131))       # 32 .. 4160
        inter = 32 * int(rng.integers(1, 66))      # 32 .. 2080
        E = int(rng.choice([1, 2, 3, 8, 16, 33, 64, 128, 260]))
        if E * hid * inter <= (1 << 26):
            break
    k = int(rng.integers(1, min(E, 16) + 1))
    T = int(rng.choice([1, 2, 3, 5, 7, 9, 15, 16, 17, 40, 64, 80]))
    logits_given = bool(rng.integers(2))
    return dtype, hid, inter, E, k, T, logits_given


CASES = list(range(48))


@pytest.mark.parametrize("seed", CASES)
def test_random_layer_shape(ctx, seed):
    dtype, hid, inter, E, k, T, logits_given = draw(1000 + seed)
    L = O.OracleMoe.synthetic(dtype, hid, inter, E, k, normalize_topk=bool(seed % 3),
                              seed=seed, with_router=not logits_given)
    router = None
    if L.router is not None:
        router = H.WeightMatrix.new(ctx, E, hid, "f32", L.router.view(np.uint8))
    moe = H.MoeLayer(ctx, seed, E, hid, inter, L.dtype, k, L.normalize, router)
    for e in range(E):
        moe.set_expert(e, L.gate[e], L.up[e], L.down[e])
    xs = O.normal(2000 + seed, T * hid).reshape(T, hid)
    logits = O.normal(3000 + seed, T * E, 0.0, 2.0).reshape(T, E) if logits_given else None
    out, idx, w = moe.forward(xs, logits=logits, return_routes=True)
    for t in range(T):
        o, i, ww = L.forward(xs[t], logits=None if logits is None else logits[t], nthreads=8)
        assert list(idx[t]) == list(i), (seed, t)
        assert same_bits(w[t], ww), (seed, t)
        assert rel_l2(out[t], o) <= REL_L2, (seed, t)
        assert same_bits(out[t], o), (seed, t)
    moe.close()
